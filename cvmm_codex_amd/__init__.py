"""cvmm_codex_amd: MI355X (gfx950) CVMM -- the routed grouped GEMM of MoE
projections -- as hand-written HIP kernels behind the reference's Python API.

    from cvmm_codex_amd import cvmm, cvmm_prepare_sel2, CVMMSel, CVMM
"""
from .api import (  # noqa: F401
    CVMM,
    CVMMSel,
    create_kernels,
    cvmm,
    cvmm_expert_offsets,
    cvmm_gate_logits,
    cvmm_gelu,
    cvmm_prepare_sel,
    cvmm_prepare_sel2,
    cvmm_route_topk,
    cvmm_triton_call,
    dtype_to_type_id,
    get_dtype,
)

__version__ = "0.1.0"
