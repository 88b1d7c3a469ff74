"""tokamak_amd -- MI355X (gfx950) attention hot path behind the Tokamak tkm.h runtime.

The product is libtkm_attn.so (HIP kernels + the C ABI in include/tkm_attn.h);
this package builds it (tokamak_amd.build) and binds it for Python callers
(tokamak_amd.attn).
"""
from .attn import (AttnError, BF16, BWD_DELTA, BWD_DKDV, BWD_DQ, BWD_DQ_DELTA, F16, attention_flops,
                   bwd_workspace_bytes, default_scale, gqa_bwd, gqa_fwd)

__all__ = ["AttnError", "BF16", "BWD_DELTA", "BWD_DKDV", "BWD_DQ", "BWD_DQ_DELTA", "F16", "attention_flops",
           "bwd_workspace_bytes", "default_scale", "gqa_bwd", "gqa_fwd"]
