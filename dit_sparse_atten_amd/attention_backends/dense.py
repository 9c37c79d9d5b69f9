"""Dense attention backend on the libdsa block-sparse kernel with a full route.

Mirrors ``DenseBackend`` of the reference (attention_backends/dense.py:12-48):
same name, call signature, dropout (``dropout_p`` on the attention
probabilities, as SDPA applies it), dtype handling (compute in ``dtype``:
bfloat16, float16 or float32, and return the caller's dtype) and output layout
(contiguous [B, T, H, D]).  The reference calls SDPA; here the same
hand-written HIP kernel as the sparse path runs with every key block listed,
so dense and sparse numerics agree by construction (float32 runs the fp32
matrix-core kernel).
"""

from __future__ import annotations

import torch

from .. import ops
from .context import install_wan_context


class DenseBackend:
    name = "dense"

    def __call__(
        self,
        q,
        k,
        v,
        q_lens=None,
        k_lens=None,
        dropout_p=0.0,
        softmax_scale=None,
        q_scale=None,
        causal=False,
        window_size=(-1, -1),
        deterministic=False,
        dtype=torch.bfloat16,
        version=None,
        **_,
    ):
        del q_lens, k_lens, deterministic, version
        if window_size != (-1, -1):
            raise NotImplementedError("The dense backend only supports global attention")
        ops.dtype_code(dtype, attention=True)  # bfloat16, float16 or float32
        output_dtype = q.dtype
        q = q.to(dtype)
        k = k.to(dtype)
        v = v.to(dtype)
        if q_scale is not None:
            q = q * q_scale
        # dropout_p > 0: SDPA's dropout on the probabilities, drawn from a
        # Philox stream seeded from torch's generator (not torch's own stream).
        output = ops.bsa_fwd(q, k, v, scale=softmax_scale, causal=causal,
                             dropout_p=float(dropout_p))
        return output.to(output_dtype)


def install(backend=None):
    """Install a backend into Wan's module-level attention call sites."""
    import wan.modules.attention as attention_module
    import wan.modules.model as model_module

    install_wan_context()
    backend = backend or DenseBackend()
    attention_module.flash_attention = backend
    model_module.flash_attention = backend
    return backend
