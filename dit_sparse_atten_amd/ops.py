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


# The 16-bit element types every kernel computes in (dtype codes of dsa.h).
KERNEL_DTYPES = {torch.bfloat16: _lib.DSA_DTYPE_BF16, torch.float16: _lib.DSA_DTYPE_F16}
# The attention (bsa_fwd, bsa_fwd_tile_stats) also computes in float32.
ATTENTION_DTYPES = {**KERNEL_DTYPES, torch.float32: _lib.DSA_DTYPE_F32}


def dtype_code(dtype, attention=False):
    """The libdsa dtype code of a torch dtype; ValueError for any other than
    bfloat16 and float16, or also float32 for the attention
    (``attention=True``)."""
    table = ATTENTION_DTYPES if attention else KERNEL_DTYPES
    if dtype not in table:
        kinds = "bfloat16, float16 or float32" if attention else "bfloat16 or float16"
        raise ValueError(f"libdsa computes in {kinds} here, not {dtype}")
    return table[dtype]


def _kernel_view(name, tensor, dtype=None, attention=False):
    """Return a [B,T,H,D] view the kernel can read (copying only if needed);
    ``dtype``, when given, is the element type every operand must share."""
    _require_cuda(name, tensor)
    if tensor.ndim != 4:
        raise ValueError(f"{name} must have shape [batch, tokens, heads, head_dim]")
    dtype_code(tensor.dtype, attention)
    if dtype is not None and tensor.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} like q, got {tensor.dtype}")
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

    def nnz_value(self):
        """Total number of routed blocks (one 8-byte device-to-host read)."""
        return int(self.nnz.item())

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
    """RouteCSR of a boolean route [H,Q,K] or [R,H,Q,K] on the device.

    Column indices are the ascending selected key blocks of each row, i.e. the
    selected prefix of the reference's stable packing
    (attention_backends/layout_ops.py:128-151); built by the HIP CSR kernels.
    """
    return route_to_csr(route, block_size=block_size)


def bsa_fwd(q, k, v, csr=None, scale=None, out=None, return_lse=False, block_size=128,
            causal=False, deterministic=False, dropout_p=0.0, seed=None, offset=0):
    """Block-sparse (or, with ``csr=None``, dense) attention forward on the GPU.

    ``block_size`` (1..128) is the number of consecutive tokens per query
    block and per key block that the route addresses: 128 for ``flex_reuse``,
    the spatial tile size for the matrix-sparse backend.

    q: [B,Tq,H,D], k/v: [B,Tk,H,D], D a multiple of 8 up to 256, all bf16,
    all fp16 or all fp32 (the compute type; fp32, and D above 128 for every
    type, run the fp32 matrix-core kernel), on a HIP device, any strides with
    a contiguous head dim.
    ``causal`` (dense calls only): query t attends keys k <= t, as SDPA's
    is_causal.  ``deterministic`` (or
    ``torch.use_deterministic_algorithms(True)``): results reproducible bit
    for bit; otherwise a routed call may start each row's key walk where the
    other rows of its head are reading (better L2 reuse), which changes the
    fp32 accumulation order and so the last bits from run to run.
    ``dropout_p`` in (0, 1) (dense calls only): dropout on the attention
    probabilities, as SDPA's ``dropout_p``, computed in fp32 with a
    Philox4x32-10 mask drawn from ``seed`` (default: a seed from torch's CPU
    generator) and ``offset`` (dsa_bsa_fwd_dropout).  Returns O [B,Tq,H,D]
    in the input type (contiguous unless ``out`` is given) and, with
    ``return_lse``, the natural-log LSE [B,H,Tq] fp32 (of the undropped
    softmax).
    """
    lib = _lib.load()
    q = _kernel_view("q", q, attention=True)
    k = _kernel_view("k", k, q.dtype, attention=True)
    v = _kernel_view("v", v, q.dtype, attention=True)
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
        out = torch.empty((batch, q_tokens, heads, head_dim), dtype=q.dtype, device=q.device)
    else:
        _require_cuda("out", out)
        if out.shape != (batch, q_tokens, heads, head_dim) or out.dtype != q.dtype:
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
    if dropout_p:
        if csr is not None:
            raise ValueError("dropout takes dense attention only")
        if not 0.0 < dropout_p < 1.0:
            raise ValueError(f"dropout_p must be in (0, 1), got {dropout_p}")
        if seed is None:
            seed = int(torch.randint(0, 2 ** 63 - 1, (), dtype=torch.int64).item())
        with torch.cuda.device(q.device):
            status = lib.dsa_bsa_fwd_dropout(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                dtype_code(q.dtype, attention=True), strides, batch, q_tokens, kv_tokens,
                heads, head_dim, float(scale), int(bool(causal)), float(dropout_p),
                int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 32 - 1),
                lse.data_ptr() if lse is not None else None, _stream_handle(q.device))
        _lib.check(status, "dsa_bsa_fwd_dropout")
        return (out, lse) if return_lse else out
    if not 1 <= block_size <= 128:
        raise ValueError(f"block_size {block_size} unsupported (1..128)")
    deterministic = bool(deterministic) or torch.are_deterministic_algorithms_enabled()
    # Room for the split partials of the last round of workgroups (none when
    # the key range is too short to split; the fp32-compute kernel, which
    # also takes head dims above 128, uses none); the caching allocator
    # recycles it.
    fp32_kernel = q.dtype == torch.float32 or head_dim > HEAD_DIM
    workspace_bytes = 0 if fp32_kernel else lib.dsa_bsa_workspace_bytes_block(
        batch, heads, kv_tokens, head_dim, block_size)
    workspace = (torch.empty(workspace_bytes, dtype=torch.uint8, device=q.device)
                 if workspace_bytes else None)
    with torch.cuda.device(q.device):
        status = lib.dsa_bsa_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            dtype_code(q.dtype, attention=True), strides,
            batch, q_tokens, kv_tokens, heads, head_dim, block_size,
            row_ptr.data_ptr() if row_ptr is not None else None,
            col_idx.data_ptr() if col_idx is not None else None,
            route_batches, float(scale), int(bool(causal)), int(bool(deterministic)),
            lse.data_ptr() if lse is not None else None,
            workspace.data_ptr() if workspace is not None else None, workspace_bytes,
            _stream_handle(q.device))
    _lib.check(status, "dsa_bsa_fwd")
    return (out, lse) if return_lse else out


def _require_bool_route(route):
    _require_cuda("route", route)
    if route.dtype != torch.bool:
        raise ValueError("route must be a boolean tensor")
    return route.contiguous()


def sampled_block_mass(q, k, block_size, samples=2, scale=None):
    """Sampled block mass [heads, blocks, blocks] fp32 of a batch-1 call.

    Same contract as the reference's ``_sampled_block_mass``
    (attention_backends/flex.py:205-251), computed by one fused HIP kernel.
    """
    lib = _lib.load()
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("sampled route update supports batch-1 self-attention")
    if samples <= 0 or samples > block_size:
        raise ValueError("route_samples must be in [1, block_size]")
    q = _kernel_view("q", q)
    k = _kernel_view("k", k, q.dtype)
    _, tokens, heads, head_dim = q.shape
    if scale is None:
        scale = head_dim ** -0.5
    blocks = math.ceil(tokens / block_size)
    mass = torch.empty((heads, blocks, blocks), dtype=torch.float32, device=q.device)
    strides = _lib.int64_array([q.stride(1), q.stride(2), k.stride(1), k.stride(2)])
    with torch.cuda.device(q.device):
        status = lib.dsa_sampled_mass(
            q.data_ptr(), k.data_ptr(), dtype_code(q.dtype), strides, tokens, heads, head_dim, block_size,
            samples, float(scale), mass.data_ptr(), _stream_handle(q.device))
    _lib.check(status, "dsa_sampled_mass")
    return mass


def block_mass(q, k, lse, block_size=128, scale=None):
    """Exact block attention mass [heads, blocks, blocks] fp32 of a batch-1 call.

    Same contract as the reference's ``_block_attention_mass``
    (attention_backends/flex.py:158-202): ``lse`` is the natural-log
    normaliser of every query row ([1, H, T] or [H, T], as ``bsa_fwd(...,
    return_lse=True)`` returns it) and mass[h, qb, kb] sums
    exp(scale * q.k - lse) over the tokens of the two blocks.
    """
    lib = _lib.load()
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("Flex bootstrap supports batch-1 self-attention")
    if block_size != 128:
        raise ValueError("The exact mass kernel currently requires block_size=128")
    q = _kernel_view("q", q)
    k = _kernel_view("k", k, q.dtype)
    _, tokens, heads, head_dim = q.shape
    _require_cuda("lse", lse)
    if lse.dtype != torch.float32:
        raise ValueError("lse must be float32")
    if lse.ndim == 3:
        if lse.shape[0] != 1:
            raise ValueError("lse must have shape [1, heads, tokens] or [heads, tokens]")
        lse = lse[0]
    if tuple(lse.shape) != (heads, tokens):
        raise ValueError("lse must have shape [1, heads, tokens] or [heads, tokens]")
    if lse.stride(1) != 1:
        lse = lse.contiguous()
    if scale is None:
        scale = head_dim ** -0.5
    blocks = math.ceil(tokens / block_size)
    mass = torch.empty((heads, blocks, blocks), dtype=torch.float32, device=q.device)
    strides = _lib.int64_array([q.stride(1), q.stride(2), k.stride(1), k.stride(2)])
    with torch.cuda.device(q.device):
        status = lib.dsa_block_mass(
            q.data_ptr(), k.data_ptr(), dtype_code(q.dtype), strides, tokens, heads, head_dim, block_size,
            lse.data_ptr(), lse.stride(0), float(scale), mass.data_ptr(),
            _stream_handle(q.device))
    _lib.check(status, "dsa_block_mass")
    return mass


def bsa_fwd_block_mass(q, k, v, scale=None):
    """Dense attention of batch-1 self-attention q/k/v [1, T, H, D] with its
    exact 128-token block mass: returns ``(out, lse, mass)`` with ``out`` and
    ``lse`` [1, H, T] as :func:`bsa_fwd` returns them and ``mass`` as
    :func:`block_mass` does (the reference's ``_dense_bootstrap`` pair of
    dense attention and ``_block_attention_mass``, attention_backends/
    flex.py:254-272, 158-202).  With T a multiple of 128 the mass comes from
    the attention launch's own probabilities; otherwise the call runs the
    attention and then the block-mass pass (bf16 and fp16; float32 inputs
    need T a multiple of 128).
    """
    lib = _lib.load()
    q = _kernel_view("q", q, attention=True)
    k = _kernel_view("k", k, q.dtype, attention=True)
    v = _kernel_view("v", v, q.dtype, attention=True)
    batch, tokens, heads, head_dim = q.shape
    if batch != 1 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("Flex bootstrap supports batch-1 self-attention")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k and v must be on the same device")
    if scale is None:
        scale = head_dim ** -0.5
    blocks = math.ceil(tokens / 128)
    out = torch.empty((1, tokens, heads, head_dim), dtype=q.dtype, device=q.device)
    lse = torch.empty((1, heads, tokens), dtype=torch.float32, device=q.device)
    mass = torch.empty((heads, blocks, blocks), dtype=torch.float32, device=q.device)
    strides = _lib.int64_array(
        list(q.stride()[:3]) + list(k.stride()[:3]) + list(v.stride()[:3])
        + list(out.stride()[:3]))
    workspace_bytes = lib.dsa_bsa_fwd_block_mass_workspace_bytes(heads, tokens, head_dim)
    workspace = (torch.empty(workspace_bytes, dtype=torch.uint8, device=q.device)
                 if workspace_bytes else None)
    with torch.cuda.device(q.device):
        status = lib.dsa_bsa_fwd_block_mass(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            dtype_code(q.dtype, attention=True),
            strides, tokens, heads, head_dim, float(scale), lse.data_ptr(), mass.data_ptr(),
            workspace.data_ptr() if workspace is not None else None, workspace_bytes,
            _stream_handle(q.device))
    _lib.check(status, "dsa_bsa_fwd_block_mass")
    return out, lse, mass


def tile_stats(q, k, lse, tile_shape, csr=None, scale=None, centroids=True):
    """Spatial-tile attention statistics of tile-major q/k [1, T, H, 128].

    Same quantities as the reference's matrix-sparse statistics
    (attention_backends/sparse.py:184-233 with ``csr=None``, 718-750 with the
    CSR of the attended tiles): ``lse`` is the natural-log normaliser of that
    attention ([1, H, T] or [H, T]).  Returns a dict of [H, tiles, tiles]
    tensors: ``mass`` (fp32, mass / tokens), ``mass_f16`` and, with
    ``centroids``, ``centroid_q_y``, ``centroid_q_x``, ``centroid_k_y``,
    ``centroid_k_x`` (fp16).
    """
    lib = _lib.load()
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("tile statistics support batch-1 self-attention")
    q = _kernel_view("q", q)
    k = _kernel_view("k", k, q.dtype)
    _, tokens, heads, head_dim = q.shape
    tile_h, tile_w = (int(x) for x in tile_shape)
    tile = tile_h * tile_w
    if tile <= 0 or tokens % tile:
        raise ValueError("the tile shape must divide the token count")
    tiles = tokens // tile
    _require_cuda("lse", lse)
    if lse.dtype != torch.float32:
        raise ValueError("lse must be float32")
    if lse.ndim == 3:
        lse = lse[0]
    if tuple(lse.shape) != (heads, tokens):
        raise ValueError("lse must have shape [1, heads, tokens] or [heads, tokens]")
    if lse.stride(1) != 1:
        lse = lse.contiguous()
    if scale is None:
        scale = head_dim ** -0.5
    row_ptr = col_idx = None
    if csr is not None:
        if (csr.route_batches, csr.heads, csr.q_blocks, csr.k_blocks) != (1, heads, tiles, tiles):
            raise ValueError("route shape does not match the tile layout")
        row_ptr, col_idx = csr.row_ptr, csr.col_idx
    shape = (heads, tiles, tiles)
    out = {"mass": torch.empty(shape, dtype=torch.float32, device=q.device),
           "mass_f16": torch.empty(shape, dtype=torch.float16, device=q.device)}
    names = ("centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x")
    if centroids:
        for name in names:
            out[name] = torch.empty(shape, dtype=torch.float16, device=q.device)
    strides = _lib.int64_array([q.stride(1), q.stride(2), k.stride(1), k.stride(2)])
    with torch.cuda.device(q.device):
        status = lib.dsa_tile_stats(
            q.data_ptr(), k.data_ptr(), dtype_code(q.dtype), strides, tokens, heads, head_dim, tile_h, tile_w,
            lse.data_ptr(), lse.stride(0),
            row_ptr.data_ptr() if row_ptr is not None else None,
            col_idx.data_ptr() if col_idx is not None else None, float(scale),
            out["mass"].data_ptr(), out["mass_f16"].data_ptr(),
            *[out[name].data_ptr() if name in out else None for name in names],
            _stream_handle(q.device))
    _lib.check(status, "dsa_tile_stats")
    return out


def bsa_fwd_tile_stats(q, k, v, csr, tile_shape, scale=None, deterministic=False,
                       centroids=True):
    """One matrix-sparse step: attention of tile-major q/k/v [1, T, H, D] over
    the CSR of kept tiles (``csr=None``: every tile, dense) and the statistics
    of that same softmax (the reference's ``sparse_chunk``, attention_backends/
    sparse.py:670-751; dense: ``_dense_route``, 184-233).  Returns
    ``(out, lse, stats)`` with ``out`` as :func:`bsa_fwd` returns it, ``lse``
    [1, H, T] and ``stats`` as :func:`tile_stats` returns them.  Every call
    gets its statistics from the attention launch itself (per query row and
    key tile), which a short second launch combines per cell; no second QK
    pass runs.  ``deterministic`` as in :func:`bsa_fwd`: without it (and
    without torch's deterministic mode) a routed call's output, mass and
    centroids can differ in the last bits from run to run.
    """
    lib = _lib.load()
    q = _kernel_view("q", q, attention=True)
    k = _kernel_view("k", k, q.dtype, attention=True)
    v = _kernel_view("v", v, q.dtype, attention=True)
    batch, tokens, heads, head_dim = q.shape
    if batch != 1 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("tile statistics support batch-1 self-attention")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k and v must be on the same device")
    tile_h, tile_w = (int(x) for x in tile_shape)
    tile = tile_h * tile_w
    if tile <= 0 or tile > 128 or tokens % tile:
        raise ValueError("the tile shape must divide the token count (1..128 tokens per tile)")
    tiles = tokens // tile
    if csr is not None:
        if (csr.route_batches, csr.heads, csr.q_blocks, csr.k_blocks, csr.block_size) != (
                1, heads, tiles, tiles, tile):
            raise ValueError("route shape does not match the tile layout")
        if csr.row_ptr.device != q.device or csr.col_idx.device != q.device:
            raise ValueError("route must live on the attention device")
        entries = csr.nnz_value() if csr.nnz is not None else int(csr.row_ptr[-1].item())
    else:
        entries = heads * tiles * tiles
    if scale is None:
        scale = head_dim ** -0.5
    deterministic = bool(deterministic) or torch.are_deterministic_algorithms_enabled()
    out = torch.empty((1, tokens, heads, head_dim), dtype=q.dtype, device=q.device)
    lse = torch.empty((1, heads, tokens), dtype=torch.float32, device=q.device)
    shape = (heads, tiles, tiles)
    stats = {"mass": torch.empty(shape, dtype=torch.float32, device=q.device),
             "mass_f16": torch.empty(shape, dtype=torch.float16, device=q.device)}
    names = ("centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x")
    if centroids:
        for name in names:
            stats[name] = torch.empty(shape, dtype=torch.float16, device=q.device)
    strides = _lib.int64_array(
        list(q.stride()[:3]) + list(k.stride()[:3]) + list(v.stride()[:3])
        + list(out.stride()[:3]))
    workspace_bytes = lib.dsa_bsa_fwd_tile_stats_workspace_bytes(
        heads, tokens, head_dim, tile_h, tile_w, entries)
    workspace = (torch.empty(workspace_bytes, dtype=torch.uint8, device=q.device)
                 if workspace_bytes else None)
    with torch.cuda.device(q.device):
        status = lib.dsa_bsa_fwd_tile_stats(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            dtype_code(q.dtype, attention=True), strides, tokens, heads, head_dim, tile_h, tile_w,
            csr.row_ptr.data_ptr() if csr is not None else None,
            csr.col_idx.data_ptr() if csr is not None else None,
            entries, float(scale), int(bool(deterministic)),
            lse.data_ptr(), stats["mass"].data_ptr(), stats["mass_f16"].data_ptr(),
            *[stats[name].data_ptr() if name in stats else None for name in names],
            workspace.data_ptr() if workspace is not None else None, workspace_bytes,
            _stream_handle(q.device))
    _lib.check(status, "dsa_bsa_fwd_tile_stats")
    return out, lse, stats


def route_select(mass, target, keep, previous=None, persistence=0.0, sink_blocks=0):
    """Prior + top-mass selection + sink on the GPU.

    mass: fp32 [..., K] (non-negative); previous: bool of the same shape or
    None.  Returns (route bool [..., K], counts int32 [...]).  The cap is
    max(1, ceil(K * keep)) exactly as the reference's ``_top_mass_route``
    (attention_backends/flex.py:83-94).
    """
    lib = _lib.load()
    _require_cuda("mass", mass)
    if mass.dtype != torch.float32:
        raise ValueError("mass must be float32")
    if not 0 < keep <= 1:
        raise ValueError("keep must be in (0, 1]")
    if not 0 < target <= 1:
        raise ValueError("mass_target must be in (0, 1]")
    mass = mass.contiguous()
    keys = mass.shape[-1]
    rows = mass.numel() // keys
    cap = max(1, math.ceil(keys * keep))
    prev_ptr = None
    if previous is not None and persistence:
        previous = _require_bool_route(previous)
        if previous.shape != mass.shape:
            raise ValueError("previous route must match the mass shape")
        prev_ptr = previous.data_ptr()
    route = torch.empty(mass.shape, dtype=torch.bool, device=mass.device)
    counts = torch.empty(mass.shape[:-1], dtype=torch.int32, device=mass.device)
    with torch.cuda.device(mass.device):
        status = lib.dsa_route_select(
            mass.data_ptr(), prev_ptr, rows, keys, float(persistence), float(target), cap,
            int(sink_blocks), route.data_ptr(), counts.data_ptr(), _stream_handle(mass.device))
    _lib.check(status, "dsa_route_select")
    return route, counts


def _neighbor_table(neighbors, blocks, device):
    _require_cuda("neighbors", neighbors)
    if tuple(neighbors.shape) != (blocks, 4):
        raise ValueError("neighbors must have shape [blocks, 4]")
    if neighbors.device != device:
        raise ValueError("neighbors must live on the route device")
    return neighbors.to(torch.int32).contiguous()


def frontier_mask(route, neighbors, return_count=False):
    """Selected route cells with an unselected valid neighbour along the query
    or key axis (attention_backends/routing.py:35-41).  route: bool [H, B, B];
    neighbors: int [B, 4] (-1 = none).  With ``return_count`` also returns the
    number of frontier cells as a device int64 tensor."""
    lib = _lib.load()
    route = _require_bool_route(route)
    if route.ndim != 3 or route.shape[1] != route.shape[2]:
        raise ValueError("route must have shape [heads, blocks, blocks]")
    heads, blocks, _ = route.shape
    neighbors = _neighbor_table(neighbors, blocks, route.device)
    frontier = torch.empty_like(route)
    count = torch.empty(1, dtype=torch.int64, device=route.device) if return_count else None
    with torch.cuda.device(route.device):
        status = lib.dsa_frontier_mask(
            route.data_ptr(), heads, blocks, neighbors.data_ptr(), frontier.data_ptr(),
            count.data_ptr() if count is not None else None, _stream_handle(route.device))
    _lib.check(status, "dsa_frontier_mask")
    return (frontier, count) if return_count else frontier


def directional_update(mass, previous, neighbors, *, keep, persistence=0.5, min_ratio=0.0,
                       candidate_bonus=0.0, budget_scale=1.0, exploration_fraction=0.0,
                       expand_q=True, expand_k=True, expand_joint=True,
                       previous_frontier=None, sink_blocks=0):
    """Frontier-aware directional route update on the GPU.

    Same contract as the reference's ``directional_budget_update``
    (attention_backends/routing.py:92-168), followed by the first
    ``sink_blocks`` columns (flex.py:544-546).  Returns a dict with route
    (after the sink), counts (int32 [H, B], sink included), candidates,
    exploration, dropped and added (the last two before the sink, as the
    reference reports them).
    """
    lib = _lib.load()
    _require_cuda("mass", mass)
    if mass.dtype != torch.float32:
        raise ValueError("mass must be float32")
    previous = _require_bool_route(previous)
    if previous.shape != mass.shape:
        raise ValueError("previous route and mass must have identical shapes")
    if mass.ndim != 3 or mass.shape[1] != mass.shape[2]:
        raise ValueError("mass must have shape [heads, blocks, blocks]")
    if budget_scale <= 0:
        raise ValueError("budget_scale must be positive")
    if not 0 <= exploration_fraction <= 1:
        raise ValueError("exploration_fraction must be in [0, 1]")
    heads, blocks, _ = mass.shape
    mass = mass.contiguous()
    neighbors = _neighbor_table(neighbors, blocks, mass.device)
    if previous_frontier is not None:
        previous_frontier = _require_bool_route(previous_frontier)
        if previous_frontier.shape != mass.shape:
            raise ValueError("previous_frontier must match the route shape")
    cap = max(1, math.ceil(blocks * keep))
    explore = max(1, math.ceil(blocks * exploration_fraction)) if exploration_fraction else 0
    flags = (1 if expand_q else 0) | (2 if expand_k else 0) | (4 if expand_joint else 0)
    outputs = {name: torch.empty(mass.shape, dtype=torch.bool, device=mass.device)
               for name in ("route", "candidates", "exploration", "dropped", "added")}
    counts = torch.empty((heads, blocks), dtype=torch.int32, device=mass.device)
    with torch.cuda.device(mass.device):
        status = lib.dsa_directional_update(
            mass.data_ptr(), previous.data_ptr(),
            previous_frontier.data_ptr() if previous_frontier is not None else None,
            neighbors.data_ptr(), heads, blocks, cap, float(persistence), float(min_ratio),
            float(candidate_bonus), float(budget_scale), explore, flags, int(sink_blocks),
            outputs["route"].data_ptr(), counts.data_ptr(), outputs["candidates"].data_ptr(),
            outputs["exploration"].data_ptr(), outputs["dropped"].data_ptr(),
            outputs["added"].data_ptr(), _stream_handle(mass.device))
    _lib.check(status, "dsa_directional_update")
    outputs["counts"] = counts
    return outputs


def drop_low_mass(mask, mass, drop_factor, sink_tiles=0):
    """Next route of the matrix-sparse backend (attention_backends/sparse.py:
    327-348, then the first ``sink_tiles`` columns): returns (route bool, counts
    int32).  ``mass`` is fp16 (the stored route mass) or fp32."""
    lib = _lib.load()
    mask = _require_bool_route(mask)
    _require_cuda("mass", mass)
    if mask.ndim != 3 or mask.shape[1] != mask.shape[2] or mass.shape != mask.shape:
        raise ValueError("mask and mass must have shape [heads, tiles, tiles]")
    if mass.dtype not in (torch.float16, torch.float32):
        raise ValueError("mass must be float16 or float32")
    heads, tiles, _ = mask.shape
    mass = mass.contiguous()
    out = torch.empty_like(mask)
    counts = torch.empty((heads, tiles), dtype=torch.int32, device=mask.device)
    scratch = torch.empty(4 * heads, dtype=torch.float32, device=mask.device)
    with torch.cuda.device(mask.device):
        status = lib.dsa_drop_low_mass(
            mask.data_ptr(), mass.data_ptr(), int(mass.dtype == torch.float16), heads, tiles,
            float(drop_factor), int(sink_tiles), scratch.data_ptr(), out.data_ptr(),
            counts.data_ptr(), _stream_handle(mask.device))
    _lib.check(status, "dsa_drop_low_mass")
    return out, counts


EXPAND_POLICIES = {"all": 1, "directional": 2}


def expand_route(mask, grid_tiles, policy, mass=None, centroids=None, centroid_threshold=0.15,
                 huge_factor=2.0):
    """Predicted next mask (attention_backends/sparse.py:350-373) for policy
    "all" or "directional".  ``grid_tiles`` = (frames, blocks_h, blocks_w);
    ``mass`` and ``centroids`` (q_y, q_x, k_y, k_x) are fp16 [H, tiles, tiles]."""
    lib = _lib.load()
    if policy not in EXPAND_POLICIES:
        raise ValueError(f"unknown expansion policy {policy!r}")
    mask = _require_bool_route(mask)
    heads, tiles, _ = mask.shape
    frames, blocks_h, blocks_w = (int(x) for x in grid_tiles)
    if frames * blocks_h * blocks_w != tiles:
        raise ValueError("the tile grid does not match the route")
    pointers = [None] * 5
    scratch = None
    if policy == "directional":
        tensors = [mass, *centroids]
        for tensor in tensors:
            _require_cuda("mass/centroid", tensor)
            if tensor.dtype != torch.float16 or tensor.shape != mask.shape:
                raise ValueError("directional expansion needs fp16 mass and centroids")
        tensors = [tensor.contiguous() for tensor in tensors]
        pointers = [tensor.data_ptr() for tensor in tensors]
        scratch = torch.empty(4 * heads, dtype=torch.float32, device=mask.device)
    out = torch.empty_like(mask)
    with torch.cuda.device(mask.device):
        status = lib.dsa_expand_route(
            mask.data_ptr(), *pointers, heads, frames, blocks_h, blocks_w,
            EXPAND_POLICIES[policy], float(centroid_threshold), float(huge_factor),
            scratch.data_ptr() if scratch is not None else None, out.data_ptr(),
            _stream_handle(mask.device))
    _lib.check(status, "dsa_expand_route")
    return out


def route_to_csr(route, counts=None, block_size=128):
    """GPU CSR of a boolean route [H,Q,K] or [R,H,Q,K] (ascending key blocks)."""
    lib = _lib.load()
    route = _require_bool_route(route)
    if route.ndim == 3:
        route = route.unsqueeze(0)
    if route.ndim != 4:
        raise ValueError("route must have shape [heads, Q, K] or [batch, heads, Q, K]")
    route_batches, heads, q_blocks, k_blocks = route.shape
    rows = route_batches * heads * q_blocks
    device = route.device
    counts_out = None
    if counts is None:
        counts_out = torch.empty((route_batches, heads, q_blocks), dtype=torch.int32,
                                 device=device)
    else:
        counts = counts.reshape(route_batches, heads, q_blocks).to(torch.int32).contiguous()
    row_ptr = torch.empty(rows + 1, dtype=torch.int32, device=device)
    col_idx = torch.empty(max(1, route.numel()), dtype=torch.int32, device=device)
    nnz = torch.empty(1, dtype=torch.int64, device=device)
    with torch.cuda.device(device):
        status = lib.dsa_route_to_csr(
            route.data_ptr(), rows, k_blocks,
            counts.data_ptr() if counts is not None else None,
            counts_out.data_ptr() if counts_out is not None else None,
            row_ptr.data_ptr(), col_idx.data_ptr(), nnz.data_ptr(), _stream_handle(device))
    _lib.check(status, "dsa_route_to_csr")
    return RouteCSR(row_ptr, col_idx, counts if counts is not None else counts_out,
                    route_batches, heads, q_blocks, k_blocks, block_size, nnz=nnz,
                    route=route)


def pack_rows(route):
    """(counts int32 [...], indices int32 [..., K]): selected ids ascending,
    then unselected ids ascending (layout_ops.py:128-151 semantics)."""
    lib = _lib.load()
    route = _require_bool_route(route)
    if route.ndim < 2:
        raise ValueError("route must be a boolean tensor with at least two axes")
    keys = route.shape[-1]
    rows = route.numel() // keys
    counts = torch.empty(route.shape[:-1], dtype=torch.int32, device=route.device)
    indices = torch.empty(route.shape, dtype=torch.int32, device=route.device)
    with torch.cuda.device(route.device):
        status = lib.dsa_pack_rows(route.data_ptr(), rows, keys, counts.data_ptr(),
                                   indices.data_ptr(), _stream_handle(route.device))
    _lib.check(status, "dsa_pack_rows")
    return counts, indices


def permute_tokens(tensors, permutation, out=None, head_major=False):
    """Gather along the token axis: out[n][b, t] = tensors[n][b, permutation[t]].

    tensors: 1-3 CUDA tensors [B, T, H, D] sharing shape and dtype, any
    strides with a contiguous last axis.  permutation: int32 [T] on the device.
    Outputs are [B, T, H, D]; contiguous, or views of head-major (BHSD)
    storage with ``head_major=True``.  Bit-exact.
    """
    lib = _lib.load()
    tensors = list(tensors)
    if not 1 <= len(tensors) <= 3:
        raise ValueError("permute_tokens moves 1 to 3 tensors")
    first = tensors[0]
    for index, tensor in enumerate(tensors):
        _require_cuda(f"tensor {index}", tensor)
        if tensor.shape != first.shape or tensor.dtype != first.dtype:
            raise ValueError("tensors must share shape and dtype")
        if tensor.ndim != 4:
            raise ValueError("tensors must have shape [batch, tokens, heads, dim]")
    _require_cuda("permutation", permutation)
    if permutation.ndim != 1 or permutation.numel() != first.shape[1]:
        raise ValueError("permutation must contain one index per token")
    permutation = permutation.to(torch.int32).contiguous()
    batch, tokens, heads, dim = first.shape
    element = first.element_size()
    sources = []
    for tensor in tensors:
        ok = (tensor.stride(3) == 1
              and all((stride * element) % 16 == 0 for stride in tensor.stride()[:3])
              and tensor.data_ptr() % 16 == 0)
        sources.append(tensor if ok else tensor.contiguous())
    if out is None:
        if head_major:
            out = [torch.empty((batch, heads, tokens, dim), dtype=first.dtype,
                               device=first.device).transpose(1, 2) for _ in sources]
        else:
            out = [torch.empty_like(first, memory_format=torch.contiguous_format)
                   for _ in sources]
    if (dim * element) % 16 != 0:
        raise ValueError("rows must be a multiple of 16 bytes")
    src_strides = _lib.int64_array(
        [s * element for tensor in sources for s in tensor.stride()[:3]])
    dst_strides = _lib.int64_array(
        [s * element for tensor in out for s in tensor.stride()[:3]])
    with torch.cuda.device(first.device):
        status = lib.dsa_permute_rows(
            len(sources), _lib.pointer_array([t.data_ptr() for t in sources]),
            _lib.pointer_array([t.data_ptr() for t in out]), src_strides, dst_strides,
            permutation.data_ptr(), batch, tokens, heads, dim * element,
            _stream_handle(first.device))
    _lib.check(status, "dsa_permute_rows")
    return out


# ---------------------------------------------------------------------------
# Wan DiT block elementwise work (end-to-end loop)
# ---------------------------------------------------------------------------

def _rows_view(name, x):
    _require_cuda(name, x)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")
    if x.stride(-1) != 1:
        x = x.contiguous()
    dim = x.shape[-1]
    rows = x.numel() // dim
    flat = x.reshape(rows, dim) if x.is_contiguous() else x.contiguous().reshape(rows, dim)
    return flat


def _f32_or_none(name, t, device):
    if t is None:
        return None
    _require_cuda(name, t)
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32")
    if t.device != device:
        raise ValueError(f"{name} must live on the tensor's device")
    t = t.contiguous()
    # The kernels read parameter vectors with 16-byte loads.
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _out_rows(out, x, rows, dim):
    """A [rows, dim] view of the caller's output tensor (or a new one)."""
    if out is None:
        return torch.empty((rows, dim), dtype=torch.bfloat16, device=x.device)
    if out.dtype != torch.bfloat16 or out.device != x.device or out.shape != x.shape:
        raise ValueError("out must be a bfloat16 tensor of x's shape on x's device")
    try:
        return out.view(rows, dim)
    except RuntimeError as exc:
        raise ValueError("out must be viewable as [rows, dim] rows") from exc


def _row_groups(name, t, rows, dim):
    """Rows per group of a per-group fp32 parameter [groups, dim]."""
    if t.numel() % dim or t.shape[-1] != dim:
        raise ValueError(f"{name} must be [groups, {dim}]")
    groups = t.numel() // dim
    if rows % groups:
        raise ValueError(f"{name} has {groups} groups, which do not divide {rows} rows")
    return rows // groups


def layernorm_modulate(x, shift=None, scale=None, weight=None, bias=None, eps=1e-6, out=None):
    """LN(x) [* weight + bias] [* (1 + scale) + shift] over the last axis of a
    bf16 [B, T, C] tensor; shift/scale fp32 [B, C] (one vector per batch item)."""
    lib = _lib.load()
    flat = _rows_view("x", x)
    rows, dim = flat.shape
    weight, bias, shift, scale = (_f32_or_none(n, t, x.device) for n, t in (
        ("weight", weight), ("bias", bias), ("shift", shift), ("scale", scale)))
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and t.numel() != dim:
            raise ValueError(f"{name} must hold {dim} values")
    per_group = _row_groups("scale", scale, rows, dim) if scale is not None else rows
    if shift is not None and (scale is None or shift.shape != scale.shape):
        raise ValueError("shift needs a scale of the same shape")
    rows_out = _out_rows(out, x, rows, dim)
    with torch.cuda.device(x.device):
        status = lib.dsa_layernorm_modulate(
            flat.data_ptr(), flat.stride(0), rows, dim,
            *[t.data_ptr() if t is not None else None for t in (weight, bias, shift, scale)],
            per_group, float(eps), rows_out.data_ptr(), rows_out.stride(0),
            _stream_handle(x.device))
    _lib.check(status, "dsa_layernorm_modulate")
    return out if out is not None else rows_out.view(x.shape)


def rmsnorm_rope(x, weight, head_dim=128, cos_sin=None, eps=1e-6, out=None):
    """rope(RMSNorm(x) * weight) over the last axis of bf16 [B, T, C]; cos_sin
    fp32 [T, head_dim / 2, 2] or None (no rotation)."""
    lib = _lib.load()
    flat = _rows_view("x", x)
    rows, dim = flat.shape
    weight = _f32_or_none("weight", weight, x.device)
    cos_sin = _f32_or_none("cos_sin", cos_sin, x.device)
    tokens = x.shape[-2] if x.ndim >= 2 else rows
    if weight.numel() != dim:
        raise ValueError(f"weight must hold {dim} values")
    if cos_sin is not None and cos_sin.numel() != tokens * head_dim:
        raise ValueError(f"cos_sin must be [{tokens}, {head_dim // 2}, 2]")
    rows_out = _out_rows(out, x, rows, dim)
    with torch.cuda.device(x.device):
        status = lib.dsa_rmsnorm_rope(
            flat.data_ptr(), flat.stride(0), rows, dim, head_dim, weight.data_ptr(),
            cos_sin.data_ptr() if cos_sin is not None else None, tokens, float(eps),
            rows_out.data_ptr(), rows_out.stride(0), _stream_handle(x.device))
    _lib.check(status, "dsa_rmsnorm_rope")
    return out if out is not None else rows_out.view(x.shape)


def gated_residual(x, y, gate=None, out=None):
    """x + gate * y over bf16 [B, T, C]; gate fp32 [B, C] or None (1)."""
    lib = _lib.load()
    fx = _rows_view("x", x)
    fy = _rows_view("y", y)
    if fx.shape != fy.shape:
        raise ValueError("x and y must have the same shape")
    rows, dim = fx.shape
    gate = _f32_or_none("gate", gate, x.device)
    per_group = _row_groups("gate", gate, rows, dim) if gate is not None else rows
    rows_out = _out_rows(out, x, rows, dim)
    with torch.cuda.device(x.device):
        status = lib.dsa_gated_residual(
            fx.data_ptr(), fx.stride(0), fy.data_ptr(), fy.stride(0),
            gate.data_ptr() if gate is not None else None, rows, dim, per_group,
            rows_out.data_ptr(), rows_out.stride(0), _stream_handle(x.device))
    _lib.check(status, "dsa_gated_residual")
    return out if out is not None else rows_out.view(x.shape)
