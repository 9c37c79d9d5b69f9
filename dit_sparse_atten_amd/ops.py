"""Torch-facing wrappers over the libdsa C-ABI.

Tensors are only plumbing here: device memory and the current HIP stream are
taken from PyTorch and passed as raw pointers.  Every compute call runs a
hand-written HIP kernel; there is no CPU or PyTorch fallback, and a CPU tensor
is rejected with ``ValueError``.
"""

from __future__ import annotations

import math

import torch

from . import _lib

HEAD_DIM = 128


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(name, tensor):
    if not isinstance(tensor, torch.Tensor) or not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor; libdsa has no CPU path")


def _kernel_view(name, tensor):
    """Return a [B,T,H,D] bf16 view the kernel can read (copying only if needed)."""
    _require_cuda(name, tensor)
    if tensor.ndim != 4:
        raise ValueError(f"{name} must have shape [batch, tokens, heads, head_dim]")
    if tensor.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {tensor.dtype}")
    ok = (
        tensor.stride(3) == 1
        and all(stride % 8 == 0 for stride in tensor.stride()[:3])
        and tensor.data_ptr() % 16 == 0
    )
    return tensor if ok else tensor.contiguous()


class RouteCSR:
    """Compressed block route: for every (route batch, head, query block) row,
    the ascending list of key blocks it attends to.

    This is the MI355X counterpart of the KV half of a FlexAttention
    ``BlockMask`` (``full_kv_num_blocks`` / ``full_kv_indices``,
    attention_backends/flex.py:326-338), keeping only the selected prefix.
    """

    __slots__ = ("row_ptr", "col_idx", "counts", "route_batches", "heads",
                 "q_blocks", "k_blocks", "block_size", "nnz", "_route")

    def __init__(self, row_ptr, col_idx, counts, route_batches, heads, q_blocks,
                 k_blocks, block_size, nnz=None, route=None):
        self.row_ptr = row_ptr
        self.col_idx = col_idx
        self.counts = counts
        self.route_batches = int(route_batches)
        self.heads = int(heads)
        self.q_blocks = int(q_blocks)
        self.k_blocks = int(k_blocks)
        self.block_size = int(block_size)
        self.nnz = nnz
        self._route = route

    @property
    def device(self):
        return self.row_ptr.device

    def to_route(self):
        """Dense boolean route [route_batches, heads, q_blocks, k_blocks]."""
        if self._route is not None:
            return self._route
        rows = self.route_batches * self.heads * self.q_blocks
        route = torch.zeros(rows, self.k_blocks, dtype=torch.bool, device=self.device)
        counts = self.counts.reshape(-1).long()
        row_ids = torch.repeat_interleave(torch.arange(rows, device=self.device), counts)
        route[row_ids, self.col_idx.long()] = True
        return route.reshape(self.route_batches, self.heads, self.q_blocks, self.k_blocks)


def csr_from_route(route, block_size=128):
    """Build a RouteCSR from a boolean route [H,Q,K] or [R,H,Q,K] (host-built).

    Column indices are the ascending selected key blocks of each row, i.e. the
    selected prefix of the reference's stable packing
    (attention_backends/layout_ops.py:128-151).
    """
    if route.dtype != torch.bool:
        raise ValueError("route must be boolean")
    if route.ndim == 3:
        route = route.unsqueeze(0)
    if route.ndim != 4:
        raise ValueError("route must have shape [heads, Q, K] or [batch, heads, Q, K]")
    route_batches, heads, q_blocks, k_blocks = route.shape
    flat = route.reshape(-1, k_blocks)
    counts = flat.sum(-1, dtype=torch.int32)
    row_ptr = torch.zeros(flat.shape[0] + 1, dtype=torch.int32, device=route.device)
    row_ptr[1:] = torch.cumsum(counts, 0, dtype=torch.int32)
    col_idx = torch.nonzero(flat, as_tuple=True)[1].to(torch.int32)
    return RouteCSR(row_ptr, col_idx, counts.reshape(route_batches, heads, q_blocks),
                    route_batches, heads, q_blocks, k_blocks, block_size,
                    nnz=int(col_idx.numel()), route=route)


def bsa_fwd(q, k, v, csr=None, scale=None, out=None, return_lse=False, block_size=128):
    """Block-sparse (or, with ``csr=None``, dense) attention forward on the GPU.

    q: [B,Tq,H,128], k/v: [B,Tk,H,128] bf16 on a HIP device, any strides with a
    contiguous head dim.  Returns O [B,Tq,H,128] bf16 (contiguous unless
    ``out`` is given) and, with ``return_lse``, the natural-log LSE [B,H,Tq] fp32.
    """
    lib = _lib.load()
    q = _kernel_view("q", q)
    k = _kernel_view("k", k)
    v = _kernel_view("v", v)
    batch, q_tokens, heads, head_dim = q.shape
    if k.shape[0] != batch or v.shape[0] != batch or k.shape[2] != heads or v.shape[2] != heads:
        raise ValueError("q, k and v must agree on batch and heads")
    if k.shape[1] != v.shape[1]:
        raise ValueError("k and v must have the same number of tokens")
    if k.shape[3] != head_dim or v.shape[3] != head_dim:
        raise ValueError("q, k and v must share the head dimension")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k and v must be on the same device")
    kv_tokens = k.shape[1]
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty((batch, q_tokens, heads, head_dim), dtype=torch.bfloat16,
                          device=q.device)
    else:
        _require_cuda("out", out)
        if out.shape != (batch, q_tokens, heads, head_dim) or out.dtype != torch.bfloat16:
            raise ValueError("out has the wrong shape or dtype")
    lse = None
    if return_lse:
        lse = torch.empty((batch, heads, q_tokens), dtype=torch.float32, device=q.device)
    row_ptr = col_idx = None
    route_batches = 1
    if csr is not None:
        if csr.block_size != block_size:
            raise ValueError("route block size does not match block_size")
        q_blocks = math.ceil(q_tokens / block_size)
        if (csr.heads, csr.q_blocks, csr.k_blocks) != (
                heads, q_blocks, math.ceil(kv_tokens / block_size)):
            raise ValueError("route shape does not match the attention shape")
        if csr.route_batches not in (1, batch):
            raise ValueError("route batches must be 1 or the attention batch")
        if csr.row_ptr.device != q.device or csr.col_idx.device != q.device:
            raise ValueError("route must live on the attention device")
        row_ptr, col_idx = csr.row_ptr, csr.col_idx
        route_batches = csr.route_batches
    strides = _lib.int64_array(
        list(q.stride()[:3]) + list(k.stride()[:3]) + list(v.stride()[:3])
        + list(out.stride()[:3]))
    with torch.cuda.device(q.device):
        status = lib.dsa_bsa_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), strides,
            batch, q_tokens, kv_tokens, heads, head_dim, block_size,
            row_ptr.data_ptr() if row_ptr is not None else None,
            col_idx.data_ptr() if col_idx is not None else None,
            route_batches, float(scale),
            lse.data_ptr() if lse is not None else None,
            _stream_handle(q.device))
    _lib.check(status, "dsa_bsa_fwd")
    return (out, lse) if return_lse else out
