"""hilda-kernel_amd: the hilda-kernel operator hot path on MI355X (gfx950).

Drop-in for the reference package ``kernels`` (triton-kernels/kernels/__init__.py:1-28),
restricted to the hot path: the same functional names, autograd Functions and
modules, backed by hand-written HIP kernels in ``libhilda_kernel_amd.so``.
FusedLinear-GRPO (``hilda_fused_linear_grpo_loss``) has no counterpart in the
reference: it is the GRPO loss behind the lm_head, chunked like
FusedLinearCrossEntropy.
Put ``hilda-kernel_amd/`` on ``sys.path`` and ``from kernels import ...`` as
with the reference.
"""
from .rms_norm import HildaRMSNormFunction, hilda_rms_norm, RMSNorm
from .rope import HildaRopeFunction, hilda_rope, RotaryEmbedding
from .swiglu import HildaSwiGLUFunction, hilda_swiglu, SwiGLU
from .geglu import HildaGeGLUFunction, hilda_geglu, GeGLU
from .kl_div import HildaKLDivFunction, hilda_kl_div, KLDivLoss
from .jsd import HildaJSDFunction, hilda_jsd, JSDLoss
from .fused_linear_jsd import HildaFusedLinearJSDFunction, hilda_fused_linear_jsd, FusedLinearJSDLoss
from .attn_res import HildaAttnResFunction, hilda_attn_res, AttnRes
from .cross_entropy import HildaCrossEntropyFunction, hilda_cross_entropy, CrossEntropyLoss
from .fused_add_rms_norm import HildaFusedAddRMSNormFunction, hilda_fused_add_rms_norm, FusedAddRMSNorm
from .fused_linear_cross_entropy import (HildaFusedLinearCrossEntropyFunction, hilda_fused_linear_cross_entropy,
                                         FusedLinearCrossEntropyLoss)
from .grpo_loss import HildaGRPOLossFunction, hilda_grpo_loss, GRPOLoss, fused_selective_log_softmax
from .fused_linear_grpo import HildaFusedLinearGRPOFunction, hilda_fused_linear_grpo_loss, FusedLinearGRPOLoss

__all__ = [
    "HildaRMSNormFunction", "hilda_rms_norm", "RMSNorm",
    "HildaRopeFunction", "hilda_rope", "RotaryEmbedding",
    "HildaSwiGLUFunction", "hilda_swiglu", "SwiGLU",
    "HildaGeGLUFunction", "hilda_geglu", "GeGLU",
    "HildaKLDivFunction", "hilda_kl_div", "KLDivLoss",
    "HildaJSDFunction", "hilda_jsd", "JSDLoss",
    "HildaFusedLinearJSDFunction", "hilda_fused_linear_jsd", "FusedLinearJSDLoss",
    "HildaAttnResFunction", "hilda_attn_res", "AttnRes",
    "HildaCrossEntropyFunction", "hilda_cross_entropy", "CrossEntropyLoss",
    "HildaFusedAddRMSNormFunction", "hilda_fused_add_rms_norm", "FusedAddRMSNorm",
    "HildaFusedLinearCrossEntropyFunction", "hilda_fused_linear_cross_entropy", "FusedLinearCrossEntropyLoss",
    "HildaGRPOLossFunction", "hilda_grpo_loss", "GRPOLoss", "fused_selective_log_softmax",
    "HildaFusedLinearGRPOFunction", "hilda_fused_linear_grpo_loss", "FusedLinearGRPOLoss",
]
