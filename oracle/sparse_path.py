"""CPU restatement of the reference's matrix-sparse path, sparse.py
(test infrastructure only; also the ``cpu_baseline`` leg of bench.py).

Follows attention_backends/sparse.py:
  tile-major reorder         81-103  (_SpatialTileLayout.to/from_tile_major)
  exact bootstrap route      184-233 (_dense_route; tile mass / tokens -> _row_mask)
  group index expansion      376-406 (_group_indices)
  per-chunk sparse attention 670-751 (sparse_chunk: gather selected key tiles,
                                      masked_fill(finfo.min), softmax, PV, and the
                                      tile-mass / centroid statistics it always pays)
  sparse step                794-930 (_sparse_attention, step >= 1, policy "reuse")
  next-route policies        258-373 (_spatial_neighbors, _apply_directional_steps,
                                      _preserve_one_per_row, _drop_low_mass, _expand)
  matrix-sparse state        794-930 (MatrixSparseCase: bootstrap, expansion,
                                      statistics, drop, sink, fp16 state)
All arithmetic is numpy float32, like the reference's fp32 CPU run.  Per-head
mass sums are exact fixed-point sums rounded once to fp32 (then fp16 for
fp16 mass), the same rule as the HIP kernels.
"""

from __future__ import annotations

import numpy as np

from . import route as route_oracle
from .spatial import sparse_tile_shape, tile_major_permutation

_F32_MIN = np.finfo(np.float32).min


def axis_offsets(length):
    """Normalised coordinates in [-1, 1] for one tile axis (sparse.py:141-146)."""
    positions = np.arange(length, dtype=np.float32)
    center = (length - 1) / 2
    scale = max((length - 1) / 2, 0.5)
    return ((positions - center) / scale).astype(np.float32)


def spatial_offsets(tile_shape, tile_count):
    local_y, local_x = np.meshgrid(axis_offsets(tile_shape[0]), axis_offsets(tile_shape[1]),
                                   indexing="ij")
    return np.tile(local_y.ravel(), tile_count), np.tile(local_x.ravel(), tile_count)


def group_indices(group_mask, tile):
    """Padded token indices of each group's selected tiles (sparse.py:376-406)."""
    counts = group_mask.sum(-1)
    max_selected = int(counts.max())
    if max_selected == 0:
        raise ValueError("Every sparse attention group must select at least one key tile")
    padded = np.zeros((group_mask.shape[0], max_selected), dtype=np.int64)
    for row in range(group_mask.shape[0]):
        ids = np.nonzero(group_mask[row])[0]
        padded[row, :ids.size] = ids
    valid_tiles = np.arange(max_selected)[None] < counts[:, None]
    indices = padded[:, :, None] * tile + np.arange(tile)
    valid = np.broadcast_to(valid_tiles[:, :, None], indices.shape)
    indices = np.where(valid, indices, 0)
    return indices.reshape(indices.shape[0], -1), valid.reshape(valid.shape[0], -1)


def _softmax(logits):
    logits = logits - logits.max(-1, keepdims=True)
    np.exp(logits, out=logits)
    logits /= logits.sum(-1, keepdims=True)
    return logits


def sparse_chunk(q, k, v, route_mask, tile, start, end, scale, stats=None, offsets=None):
    """Sparse attention for query tokens [start, end) of tile-major q/k/v
    ([1, T, H, D] float32).  Fills ``stats`` (mass, q_y, q_x, k_y, k_x as
    [H, tiles, tiles]) when given, as the reference's PyTorch path always does."""
    tokens, heads, head_dim = q.shape[1:]
    first = start // tile
    query_tiles = (end - start) // tile
    grouped_q = q[0, start:end].reshape(query_tiles, tile, heads, head_dim)
    grouped_q = grouped_q.transpose(0, 2, 1, 3).reshape(-1, tile, head_dim)
    group_heads = np.tile(np.arange(heads), query_tiles)
    group_mask = route_mask[:, first:first + query_tiles].transpose(1, 0, 2).reshape(
        query_tiles * heads, -1)
    padded, valid = group_indices(group_mask, tile)
    selected_k = k[0, padded, group_heads[:, None]]
    selected_v = v[0, padded, group_heads[:, None]]
    logits = np.matmul(grouped_q, selected_k.transpose(0, 2, 1))
    logits *= np.float32(scale)
    np.copyto(logits, _F32_MIN, where=~valid[:, None])
    probabilities = _softmax(logits)
    output = np.matmul(probabilities, selected_v)
    output = output.reshape(query_tiles, heads, tile, -1).transpose(0, 2, 1, 3).reshape(
        1, end - start, heads, -1)
    if stats is not None:
        tiles = stats["mass"].shape[-1]
        key_mass = probabilities.sum(1)
        key_tiles = padded // tile
        groups = query_tiles * heads
        group_mass = np.zeros((groups, tiles), dtype=np.float32)
        rows = np.repeat(np.arange(groups), key_tiles.shape[1])
        np.add.at(group_mass, (rows, key_tiles.ravel()), (key_mass * valid).ravel())
        stats["mass"][:, first:first + query_tiles] = group_mass.reshape(
            query_tiles, heads, -1).transpose(1, 0, 2)
        if offsets is None:
            offsets = (np.zeros(tokens, dtype=np.float32),
                       np.tile(axis_offsets(tile), tokens // tile))
        for axis, axis_offset in zip(("y", "x"), offsets):
            local_q = axis_offset[start:end].reshape(query_tiles, tile)
            local_q = np.repeat(local_q[:, None], heads, 1).reshape(-1, tile)
            q_key_mass = (probabilities * local_q[:, :, None]).sum(1)
            q_moment = np.zeros_like(group_mass)
            np.add.at(q_moment, (rows, key_tiles.ravel()), (q_key_mass * valid).ravel())
            local_k = axis_offset[padded]
            k_moment = np.zeros_like(group_mass)
            np.add.at(k_moment, (rows, key_tiles.ravel()), (key_mass * local_k * valid).ravel())
            stats[f"q_{axis}"][:, first:first + query_tiles] = q_moment.reshape(
                query_tiles, heads, -1).transpose(1, 0, 2)
            stats[f"k_{axis}"][:, first:first + query_tiles] = k_moment.reshape(
                query_tiles, heads, -1).transpose(1, 0, 2)
    return output


def empty_stats(heads, tiles):
    return {name: np.zeros((heads, tiles, tiles), dtype=np.float32)
            for name in ("mass", "q_y", "q_x", "k_y", "k_x")}


def dense_route(q, k, v, tile, query_chunk, target, keep, scale=None, stats=None,
                offsets=None):
    """Exact bootstrap (sparse.py:184-233): dense fp32 attention in query chunks,
    tile mass normalised by token count, then top-mass rows.  q/k/v tile-major.
    Fills ``stats`` (all five moments) when given.
    Returns (route [H, tiles, tiles], normalised mass, output)."""
    tokens, heads, head_dim = q.shape[1:]
    tiles = tokens // tile
    if scale is None:
        scale = head_dim ** -0.5
    mass = np.zeros((heads, tiles, tiles), dtype=np.float32)
    output = np.empty_like(q)
    chunk = max(tile, query_chunk // tile * tile)
    kh = k[0].transpose(1, 0, 2)
    vh = v[0].transpose(1, 0, 2)
    for start in range(0, tokens, chunk):
        end = min(start + chunk, tokens)
        qh = q[0, start:end].transpose(1, 0, 2)
        probabilities = _softmax((np.matmul(qh, kh.transpose(0, 2, 1)) * np.float32(scale))
                                 .astype(np.float32))
        output[0, start:end] = np.matmul(probabilities, vh).transpose(1, 0, 2)
        query_tiles = (end - start) // tile
        shape = (heads, query_tiles, tile, tiles, tile)
        dest = slice(start // tile, start // tile + query_tiles)
        mass[:, dest] = probabilities.reshape(shape).sum((2, 4))
        if stats is not None:
            for axis, axis_offset in zip(("y", "x"), offsets):
                stats[f"q_{axis}"][:, dest] = (probabilities * axis_offset[start:end].reshape(
                    1, -1, 1)).reshape(shape).sum((2, 4))
                stats[f"k_{axis}"][:, dest] = (probabilities * axis_offset.reshape(
                    1, 1, -1)).reshape(shape).sum((2, 4))
    if stats is not None:
        stats["mass"][...] = mass
    normalized = (mass / np.float32(tokens)).astype(np.float32)
    return route_oracle.top_mass_route(normalized, target, keep), normalized, output


class SparsePathCase:
    """The sparse.py call for one (layer, branch) on a Wan grid, restated.

    ``bootstrap()`` is the step-0 call (dense route + sink); ``step()`` is a
    later step with policy "reuse": sparse attention over the stored route
    (statistics included, as the PyTorch path computes them).
    """

    def __init__(self, grid, tile=64, keep=0.625, mass_target=0.90, query_chunk=256,
                 first_frame_sink=True):
        self.grid = tuple(int(value) for value in grid)
        tokens = self.grid[0] * self.grid[1] * self.grid[2]
        self.tile_shape = sparse_tile_shape(self.grid, tile, tokens)
        if self.tile_shape is None:
            raise ValueError("grid has no exact tile layout")
        self.tile = self.tile_shape[0] * self.tile_shape[1]
        self.block_h = self.grid[1] // self.tile_shape[0]
        self.block_w = self.grid[2] // self.tile_shape[1]
        self.permutation = tile_major_permutation(self.grid, self.tile_shape)
        self.inverse = np.empty_like(self.permutation)
        self.inverse[self.permutation] = np.arange(self.permutation.size, dtype=np.int32)
        self.keep = keep
        self.mass_target = mass_target
        self.query_chunk = query_chunk
        self.first_frame_sink = first_frame_sink
        self.route = None

    def to_tile_major(self, tensor):
        return tensor[:, self.permutation]

    def from_tile_major(self, tensor):
        return tensor[:, self.inverse]

    def bootstrap(self, q, k, v, scale=None):
        q, k, v = (self.to_tile_major(np.asarray(t, dtype=np.float32)) for t in (q, k, v))
        route, _, output = dense_route(q, k, v, self.tile, self.query_chunk,
                                       self.mass_target, self.keep, scale)
        if self.first_frame_sink:
            route[..., :self.block_h * self.block_w] = True
        self.route = route
        return self.from_tile_major(output)

    def step(self, q, k, v, scale=None, collect_stats=True):
        q, k, v = (self.to_tile_major(np.asarray(t, dtype=np.float32)) for t in (q, k, v))
        tokens, heads, head_dim = q.shape[1:]
        if scale is None:
            scale = head_dim ** -0.5
        tiles = tokens // self.tile
        stats = empty_stats(heads, tiles) if collect_stats else None
        offsets = spatial_offsets(self.tile_shape, tiles) if collect_stats else None
        output = np.empty_like(q)
        chunk = max(self.tile, self.query_chunk // self.tile * self.tile)
        for start in range(0, tokens, chunk):
            end = min(start + chunk, tokens)
            output[:, start:end] = sparse_chunk(q, k, v, self.route, self.tile, start, end,
                                                scale, stats, offsets)
        return self.from_tile_major(output)


# ---------------------------------------------------------------------------
# Next-route policies (sparse.py:258-373)
# ---------------------------------------------------------------------------

def head_sums(mask, mass):
    """Exact per-head sums of the selected (non-negative) mass, rounded once to
    fp32, and the selected counts."""
    m32 = np.where(mask, np.maximum(np.asarray(mass, dtype=np.float32), 0), 0).astype(np.float32)
    flat = m32.reshape(m32.shape[0], -1)
    return route_oracle.row_sums_f32(flat, scaled=False), mask.reshape(mask.shape[0], -1).sum(-1)


def preserve_one_per_row(kept, original, mass):
    """Rows emptied by the drop get their first highest-mass original tile
    (sparse.py:327-336)."""
    kept = kept.copy()
    empty = ~kept.any(-1) & original.any(-1)
    scores = np.where(original, np.asarray(mass, dtype=np.float64), -np.inf)
    fallback = scores.argmax(-1)
    heads, rows = np.nonzero(empty)
    kept[heads, rows, fallback[heads, rows]] = True
    return kept


def drop_low_mass(mask, mass, drop_factor):
    """sparse.py:339-348.  fp16 mass (the stored route mass) follows torch's
    fp16 evaluation: mean = fp16(sum16 / count), ratio = fp16(m / mean),
    compared with fp16(drop_factor); fp32 mass stays in fp32."""
    mask = np.asarray(mask, dtype=bool)
    if drop_factor <= 0:
        return mask
    mass = np.asarray(mass)
    sums, counts = head_sums(mask, mass)
    counts = np.maximum(counts, 1).astype(np.float32)
    if mass.dtype == np.float16:
        sum16 = sums.astype(np.float16).astype(np.float32)
        mean = (sum16 / counts).astype(np.float16).astype(np.float32)[:, None, None]
        with np.errstate(divide="ignore", invalid="ignore"):
            ratio = (mass.astype(np.float32) / mean).astype(np.float16).astype(np.float32)
        threshold = np.float32(np.float16(drop_factor))
    else:
        mean = np.maximum((sums / counts).astype(np.float32), np.float32(1e-12))[:, None, None]
        ratio = (mass.astype(np.float32) / mean).astype(np.float32)
        threshold = np.float32(drop_factor)
    with np.errstate(invalid="ignore"):
        kept = mask & (ratio >= threshold)
    return preserve_one_per_row(kept, mask, mass.astype(np.float32))


def _shift(mask, dimension, delta):
    """Shift one axis by delta without wrapping (sparse.py:246-255)."""
    out = np.zeros_like(mask)
    size = mask.shape[dimension]
    src = [slice(None)] * mask.ndim
    dst = [slice(None)] * mask.ndim
    src[dimension] = slice(max(0, -delta), size - max(0, delta))
    dst[dimension] = slice(max(0, delta), size - max(0, -delta))
    out[tuple(dst)] = mask[tuple(src)]
    return out


def spatial_neighbors(grid_mask):
    """Eight coupled query/key neighbours on [H, F, bh, bw, F, bh, bw]
    (sparse.py:258-276)."""
    out = grid_mask.copy()
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            if dy == 0 and dx == 0:
                continue
            shifted = grid_mask
            for dimension, delta in ((2, dy), (3, dx), (5, dy), (6, dx)):
                if delta:
                    shifted = _shift(shifted, dimension, delta)
            out |= shifted
    return out


def _direction(centroid, threshold):
    c = np.asarray(centroid, dtype=np.float16).astype(np.float32)
    return np.where(np.abs(c) < np.float32(np.float16(threshold)), 0, np.sign(c)).astype(np.int64)


def expand(state, policy, grid_tiles, centroid_threshold=0.15, huge_factor=2.0):
    """Predicted next mask (sparse.py:350-373); state holds mask (bool), mass
    and centroid_* (fp16) [H, tiles, tiles]."""
    mask = np.asarray(state["mask"], dtype=bool)
    if policy == "reuse":
        return mask
    heads = mask.shape[0]
    frames, bh, bw = grid_tiles
    shape7 = (heads, frames, bh, bw, frames, bh, bw)
    grid = mask.reshape(shape7)
    if policy == "all":
        return spatial_neighbors(grid).reshape(mask.shape)
    mass = np.asarray(state["mass"]).astype(np.float32)
    sums, counts = head_sums(mask, mass)
    mean = np.maximum((sums / np.maximum(counts, 1).astype(np.float32)).astype(np.float32),
                      np.float32(1e-12))[:, None, None]
    huge = mask & ((mass / mean).astype(np.float32) >= np.float32(huge_factor))
    predicted = grid | spatial_neighbors(huge.reshape(shape7))
    source = np.nonzero((mask & ~huge).reshape(shape7))
    if source[0].size:
        dirs = {name: _direction(state[f"centroid_{name}"], centroid_threshold).reshape(
            shape7)[source] for name in ("q_y", "q_x", "k_y", "k_x")}
        sizes = {2: bh, 3: bw, 5: bh, 6: bw}
        for move_q, move_k in ((True, False), (False, True), (True, True)):
            target = list(source)
            valid = np.ones(source[0].size, dtype=bool)
            moved = np.zeros(source[0].size, dtype=bool)
            dims = []
            if move_q:
                dims += [(2, "q_y"), (3, "q_x")]
            if move_k:
                dims += [(5, "k_y"), (6, "k_x")]
            for dimension, name in dims:
                target[dimension] = source[dimension] + dirs[name]
                valid &= (target[dimension] >= 0) & (target[dimension] < sizes[dimension])
                moved |= dirs[name] != 0
            valid &= moved
            predicted[tuple(index[valid] for index in target)] = True
    return predicted.reshape(mask.shape)


class MatrixSparseCase:
    """The matrix-sparse backend's per-(layer, branch) state machine
    (sparse.py:794-930), restated: step 0 runs the dense route; later steps
    expand the stored mask by the policy, run sparse attention over it
    (statistics for every policy but "reuse"), drop low-mass tiles, add the
    sink and keep fp16 mass and centroids."""

    def __init__(self, grid, tile=64, keep=0.625, mass_target=0.90, query_chunk=256,
                 policy="reuse", centroid_threshold=0.15, drop_factor=0.1, huge_factor=2.0,
                 first_frame_sink=True):
        self.case = SparsePathCase(grid, tile, keep, mass_target, query_chunk, first_frame_sink)
        self.policy = policy
        self.centroid_threshold = centroid_threshold
        self.drop_factor = drop_factor
        self.huge_factor = huge_factor
        self.state = None

    @property
    def grid_tiles(self):
        c = self.case
        return (c.grid[0], c.block_h, c.block_w)

    def _sink(self, mask):
        c = self.case
        if c.first_frame_sink:
            mask[..., :c.block_h * c.block_w] = True
        return mask

    def step(self, step, q, k, v, scale=None):
        c = self.case
        q, k, v = (c.to_tile_major(np.asarray(t, dtype=np.float32)) for t in (q, k, v))
        tokens, heads, head_dim = q.shape[1:]
        if scale is None:
            scale = head_dim ** -0.5
        tiles = tokens // c.tile
        offsets = spatial_offsets(c.tile_shape, tiles)
        stats = empty_stats(heads, tiles)
        if step == 0 or self.state is None:
            route, normalized, output = dense_route(q, k, v, c.tile, c.query_chunk,
                                                    c.mass_target, c.keep, scale, stats, offsets)
            den = np.maximum(stats["mass"], np.float32(1e-12))
            self.state = {"mask": self._sink(route), "mass": normalized.astype(np.float16)}
            for name in ("q_y", "q_x", "k_y", "k_x"):
                self.state[f"centroid_{name}"] = (stats[name] / den).astype(np.float16)
            return c.from_tile_major(output)
        previous = self.state
        route = expand(previous, self.policy, self.grid_tiles, self.centroid_threshold,
                       self.huge_factor)
        collect = self.policy != "reuse"
        output = np.empty_like(q)
        chunk = max(c.tile, c.query_chunk // c.tile * c.tile)
        for start in range(0, tokens, chunk):
            end = min(start + chunk, tokens)
            output[:, start:end] = sparse_chunk(q, k, v, route, c.tile, start, end, scale,
                                                stats if collect else None, offsets)
        if self.policy == "reuse":
            next_mask = drop_low_mass(route, previous["mass"], self.drop_factor)
            state = dict(previous)
        else:
            normalized = (stats["mass"] / np.float32(tokens)).astype(np.float32)
            next_mask = drop_low_mass(route, normalized, self.drop_factor)
            den = np.maximum(stats["mass"], np.float32(1e-12))
            state = {"mass": normalized.astype(np.float16)}
            for name in ("q_y", "q_x", "k_y", "k_x"):
                state[f"centroid_{name}"] = (stats[name] / den).astype(np.float16)
        state["mask"] = self._sink(np.array(next_mask, copy=True))
        self.state = state
        return c.from_tile_major(output)
