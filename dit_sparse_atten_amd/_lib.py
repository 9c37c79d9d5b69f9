"""ctypes binding of libdsa.so, the C-ABI of the HIP kernels.

Every call is asynchronous on the given HIP stream and returns a status code;
``check`` turns a failure into the exception type the reference raises for the
same condition (``ValueError`` for invalid arguments, ``RuntimeError`` for a
runtime failure).  There is no fallback: if the library is missing, loading
raises ``RuntimeError`` naming the build command.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libdsa.so"

DSA_OK = 0
DSA_EINVAL = -1
DSA_EUNSUPPORTED = -2
DSA_ELAUNCH = -3

# Element types of the attention inputs (DSA_DTYPE_* in dsa.h).
DSA_DTYPE_BF16 = 0
DSA_DTYPE_F16 = 1
DSA_DTYPE_F32 = 2  # the attention entry points only

_c_int = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_float = ctypes.c_float
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes).  Must match include/dsa.h exactly.
SIGNATURES = {
    "dsa_version": (_c_int, ()),
    "dsa_last_error": (ctypes.c_char_p, ()),
    "dsa_bsa_fwd": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,  # q, k, v, o, dtype
        ctypes.POINTER(_c_i64),                    # strides[12]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # batch, q_tokens, kv_tokens, heads, head_dim
        _c_int,                                    # block_size
        _c_ptr, _c_ptr, _c_int,                    # row_ptr, col_idx, route_batches
        _c_float, _c_int, _c_int, _c_ptr,          # scale, causal, deterministic, lse
        _c_ptr, _c_size, _c_ptr,                   # workspace, workspace_bytes, stream
    )),
    "dsa_bsa_fwd_noalloc": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,  # q, k, v, o, dtype
        ctypes.POINTER(_c_i64),                    # strides[12]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # batch, q_tokens, kv_tokens, heads, head_dim
        _c_int,                                    # block_size
        _c_ptr, _c_ptr, _c_int,                    # row_ptr, col_idx, route_batches
        _c_float, _c_int, _c_int, _c_ptr, _c_ptr,  # scale, causal, deterministic, lse, stream
    )),
    "dsa_bsa_fwd_dropout": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,  # q, k, v, o, dtype
        ctypes.POINTER(_c_i64),                    # strides[12]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # batch, q_tokens, kv_tokens, heads, head_dim
        _c_float, _c_int, _c_float,                # scale, causal, dropout_p
        ctypes.c_uint64, ctypes.c_uint32,          # seed, offset
        _c_ptr, _c_ptr,                            # lse, stream
    )),
    "dsa_bsa_workspace_bytes": (_c_size, (_c_int, _c_int, _c_int, _c_int)),
    "dsa_bsa_workspace_bytes_block": (_c_size, (_c_int, _c_int, _c_int, _c_int, _c_int)),
    "dsa_sampled_mass": (_c_int, (
        _c_ptr, _c_ptr, _c_int,                    # q, k, dtype
        ctypes.POINTER(_c_i64),                    # strides[4]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # tokens, heads, head_dim, block, samples
        _c_float, _c_ptr, _c_ptr,                  # scale, mass, stream
    )),
    "dsa_block_mass": (_c_int, (
        _c_ptr, _c_ptr, _c_int,                    # q, k, dtype
        ctypes.POINTER(_c_i64),                    # strides[4]
        _c_int, _c_int, _c_int, _c_int,            # tokens, heads, head_dim, block
        _c_ptr, _c_i64, _c_float, _c_ptr, _c_ptr,  # lse, lse_head_stride, scale, mass, stream
    )),
    "dsa_tile_stats": (_c_int, (
        _c_ptr, _c_ptr, _c_int,                    # q, k, dtype
        ctypes.POINTER(_c_i64),                    # strides[4]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # tokens, heads, head_dim, tile_h, tile_w
        _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_float,  # lse, lse_head_stride, row_ptr, col_idx, scale
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # mass, mass_f16, centroids q_y q_x k_y k_x
        _c_ptr,                                    # stream
    )),
    "dsa_bsa_fwd_tile_stats": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,  # q, k, v, o, dtype
        ctypes.POINTER(_c_i64),                    # strides[12]
        _c_int, _c_int, _c_int, _c_int, _c_int,    # tokens, heads, head_dim, tile_h, tile_w
        _c_ptr, _c_ptr, _c_i64,                    # row_ptr, col_idx, entries
        _c_float, _c_int, _c_ptr,                  # scale, deterministic, lse
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # mass, mass_f16, centroids q_y q_x k_y k_x
        _c_ptr, _c_size, _c_ptr,                   # workspace, workspace_bytes, stream
    )),
    "dsa_bsa_fwd_tile_stats_workspace_bytes": (_c_size, (
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64,  # heads, tokens, head_dim, tile_h, tile_w, entries
    )),
    "dsa_bsa_fwd_block_mass": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,  # q, k, v, o, dtype
        ctypes.POINTER(_c_i64),                    # strides[12]
        _c_int, _c_int, _c_int, _c_float,          # tokens, heads, head_dim, scale
        _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr,   # lse, mass, workspace, workspace_bytes, stream
    )),
    "dsa_bsa_fwd_block_mass_workspace_bytes": (_c_size, (_c_int, _c_int, _c_int)),
    "dsa_route_select": (_c_int, (
        _c_ptr, _c_ptr, _c_int, _c_int,            # mass, previous, rows, keys
        _c_float, _c_float, _c_int, _c_int,        # rho, target, cap, sink_blocks
        _c_ptr, _c_ptr, _c_ptr,                    # route, counts, stream
    )),
    "dsa_frontier_mask": (_c_int, (
        _c_ptr, _c_int, _c_int, _c_ptr,            # route, heads, blocks, neighbors
        _c_ptr, _c_ptr, _c_ptr,                    # frontier, count, stream
    )),
    "dsa_directional_update": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr,            # mass, previous, previous_frontier, neighbors
        _c_int, _c_int, _c_int,                    # heads, blocks, cap
        _c_float, _c_float, _c_float, _c_float,    # persistence, min_ratio, bonus, budget_scale
        _c_int, _c_int, _c_int,                    # explore_count, expand_flags, sink_blocks
        _c_ptr, _c_ptr, _c_ptr,                    # route, counts, candidates
        _c_ptr, _c_ptr, _c_ptr, _c_ptr,            # exploration, dropped, added, stream
    )),
    "dsa_drop_low_mass": (_c_int, (
        _c_ptr, _c_ptr, _c_int, _c_int, _c_int,    # mask, mass, mass_is_f16, heads, tiles
        _c_float, _c_int, _c_ptr, _c_ptr, _c_ptr,  # drop_factor, sink, scratch, out, counts
        _c_ptr,                                    # stream
    )),
    "dsa_expand_route": (_c_int, (
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # mask, mass, centroids q_y q_x k_y k_x
        _c_int, _c_int, _c_int, _c_int, _c_int,    # heads, frames, blocks_h, blocks_w, policy
        _c_float, _c_float, _c_ptr, _c_ptr, _c_ptr,  # threshold, huge, scratch, out, stream
    )),
    "dsa_route_to_csr": (_c_int, (
        _c_ptr, _c_int, _c_int,                    # route, rows, keys
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,    # counts, counts_out, row_ptr, col_idx, nnz
        _c_ptr,                                    # stream
    )),
    "dsa_pack_rows": (_c_int, (
        _c_ptr, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr,  # route, rows, keys, counts, indices, stream
    )),
    "dsa_permute_rows": (_c_int, (
        _c_int, ctypes.POINTER(_c_ptr), ctypes.POINTER(_c_ptr),  # tensors, src[], dst[]
        ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64),          # src/dst byte strides
        _c_ptr, _c_int, _c_int, _c_int, _c_int,                  # perm, batch, tokens, heads, row_bytes
        _c_ptr,                                                  # stream
    )),
    "dsa_layernorm_modulate": (_c_int, (
        _c_ptr, _c_i64, _c_int, _c_int,            # x, x_stride, rows, dim
        _c_ptr, _c_ptr, _c_ptr, _c_ptr,            # weight, bias, shift, scale
        _c_int, _c_float, _c_ptr, _c_i64, _c_ptr,  # rows_per_group, eps, out, out_stride, stream
    )),
    "dsa_rmsnorm_rope": (_c_int, (
        _c_ptr, _c_i64, _c_int, _c_int, _c_int,    # x, x_stride, rows, dim, head_dim
        _c_ptr, _c_ptr, _c_int, _c_float,          # weight, cos_sin, tokens, eps
        _c_ptr, _c_i64, _c_ptr,                    # out, out_stride, stream
    )),
    "dsa_gated_residual": (_c_int, (
        _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr,    # x, x_stride, y, y_stride, gate
        _c_int, _c_int, _c_int, _c_ptr, _c_i64,    # rows, dim, rows_per_group, out, out_stride
        _c_ptr,                                    # stream
    )),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load libdsa.so once and bind the signatures; raise if it is missing."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"{LIBRARY_PATH} is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python -m dit_sparse_atten_amd.csrc.build`")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(lib, name)
            function.restype = restype
            function.argtypes = list(argtypes)
        _lib = lib
        return lib


def last_error() -> str:
    message = load().dsa_last_error()
    return message.decode() if message else ""


def check(status: int, what: str) -> None:
    """Raise the reference's exception type for a failed libdsa call."""
    if status == DSA_OK:
        return
    message = last_error() or f"{what} failed with status {status}"
    if status in (DSA_EINVAL, DSA_EUNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def pointer_array(values):
    values = [int(value) for value in values]
    return (_c_ptr * len(values))(*values)


def int64_array(values):
    values = [int(value) for value in values]
    return (_c_i64 * len(values))(*values)
