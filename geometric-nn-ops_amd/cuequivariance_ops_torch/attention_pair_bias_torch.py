"""cueq's ``attention_pair_bias`` on the HIP kernels (reference shim
attention_pair_bias_torch.py:1-85; cueq deep-imports it from this module path).

``b_ln_z`` and ``b_proj_z`` add one constant per head and query row to the logits, which the
softmax cancels: they cannot change the output, so they are dropped with a warning (cueq
folds them into its returned bias, which then differs from ours by that constant).
"""

import sys
import warnings

import torch

from geometric_nn_ops_torch.triangle import attention_pair_bias as _attention_pair_bias

# cueq's documented fallback threshold (advertised, not consulted).
CUEQ_ATTENTION_PAIR_BIAS_FALLBACK_THRESHOLD = sys.maxsize


def attention_pair_bias(s: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, z: torch.Tensor,
                        mask: torch.Tensor, num_heads: int, w_proj_z: torch.Tensor | None, w_proj_g: torch.Tensor,
                        w_proj_o: torch.Tensor, w_ln_z: torch.Tensor | None = None,
                        b_ln_z: torch.Tensor | None = None, b_proj_z: torch.Tensor | None = None,
                        b_proj_g: torch.Tensor | None = None, b_proj_o: torch.Tensor | None = None,
                        inf: float = 1e6, eps: float = 1e-5, attn_scale: float | None = None,
                        return_z_proj: bool = True, is_cached_z_proj: bool = False):
    if q.shape[1] != num_heads:
        raise ValueError(f"num_heads={num_heads} does not match q head dim {q.shape[1]}")
    for name, value in (("b_ln_z", b_ln_z), ("b_proj_z", b_proj_z)):
        if value is not None:
            warnings.warn(f"{name} is ignored: it shifts every logit of a query row by the same amount, "
                          "which the softmax cancels", stacklevel=2)
    return _attention_pair_bias(s, q, k, v, z, proj_g_weight=w_proj_g, proj_o_weight=w_proj_o,
                                proj_z_weight=w_proj_z, ln_z_weight=w_ln_z, proj_g_bias=b_proj_g,
                                proj_o_bias=b_proj_o, mask=mask, scale=attn_scale, inf=inf, eps=eps,
                                z_is_projected=is_cached_z_proj, return_z_proj=return_z_proj)
