"""Gate module (reference package ``tasft/modules/__init__.py``, AttnGate part)."""
from tasft_amd.modules.attn_gate import AttnGate, GateOutput

__all__ = ["AttnGate", "GateOutput"]
