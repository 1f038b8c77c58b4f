"""MI355X-native fused FP8 block-scale MoE layer (DeepSeek-V3 routing, top-8 of 256
experts, 32 local experts, H=7168, I=2048) behind the entry point of
nikhilnd/mlsys26-flashinfer-moe's `run` (kernel.py:562-729).

The directory name contains hyphens, so import it through `load_package()` in
__graft_entry__.py, which registers it as `mlsys26_flashinfer_moe_amd`.
"""
from . import _lib
from .moe import (Workspace, clear_packed_weights, make_args, pack_weights, quantize_hidden, run, run_packed,
                  set_packed_weight_sets, validate, workspace_for)

__all__ = ["run", "run_packed", "pack_weights", "set_packed_weight_sets", "clear_packed_weights",
           "quantize_hidden", "validate", "make_args", "Workspace", "workspace_for", "_lib"]
