"""Gate-target operator (reference ``tasft/training/objectives.py:128-185``)."""
from tasft_amd.training.objectives import TASFTObjective, gate_target_from_qk

__all__ = ["TASFTObjective", "gate_target_from_qk"]
