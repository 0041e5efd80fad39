"""Gate terms of the training objective (reference ``tasft/training/objectives.py:128-240``)."""
from tasft_amd.training.objectives import TASFTObjective, gate_loss_from_qk, gate_target_from_qk

__all__ = ["TASFTObjective", "gate_loss_from_qk", "gate_target_from_qk"]
