"""Morton-ordered spatial micro-tile layout for 128-token route blocks.

Mirrors attention_backends/spatial.py of the reference:
  * micro-tile choice (spatial.py:30-43): the largest exact H x W tile whose
    area is <= max tokens and divides the block size, then the least elongated;
  * order (spatial.py:121-131): frame-major, tiles within a frame sorted by
    (Morton code, y, x), tokens row-major inside a tile;
  * 4-neighbour block table by majority vote (spatial.py:149-173) and the
    block -> frame map.
The permutation is built on the host once per grid (vectorised numpy);
reorder/restore run the libdsa gather kernel.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import layout_ops


def _microtile(height, width, block_size, max_tokens):
    best_key, best = None, (1, 1)
    for tile_h in (d for d in range(1, height + 1) if height % d == 0):
        for tile_w in (d for d in range(1, width + 1) if width % d == 0):
            area = tile_h * tile_w
            if area > max_tokens or block_size % area:
                continue
            key = (-area, abs(math.log(tile_w / tile_h)))
            if best_key is None or key < best_key:
                best_key, best = key, (tile_h, tile_w)
    return best


def _interleave_bits(ys, xs):
    """Morton code with x bits at even and y bits at odd positions."""
    code = np.zeros_like(xs)
    bits = int(max(int(ys.max(initial=0)), int(xs.max(initial=0)))).bit_length()
    for bit in range(bits):
        code |= ((xs >> bit) & 1) << (2 * bit)
        code |= ((ys >> bit) & 1) << (2 * bit + 1)
    return code


@dataclass
class SpatialTokenLayout:
    grid: tuple[int, int, int]
    block_size: int
    microtile_shape: tuple[int, int]
    permutation_cpu: torch.Tensor
    inverse_cpu: torch.Tensor
    neighbors_cpu: torch.Tensor
    block_frames_cpu: torch.Tensor

    def __post_init__(self):
        self._device_cache = {}

    @property
    def tokens(self):
        frames, height, width = self.grid
        return frames * height * width

    @property
    def blocks(self):
        return math.ceil(self.tokens / self.block_size)

    @property
    def signature(self):
        return self.grid, self.block_size, self.microtile_shape

    def _device_values(self, device):
        device = torch.device(device)
        if device not in self._device_cache:
            self._device_cache[device] = (
                self.permutation_cpu.to(device),
                self.inverse_cpu.to(device),
                self.neighbors_cpu.to(device),
            )
        return self._device_cache[device]

    def reorder(self, tensor):
        permutation, _, _ = self._device_values(tensor.device)
        return layout_ops.reorder(tensor, permutation)

    def reorder_qkv(self, q, k, v):
        """Reorder Q/K/V together in one launch (head-major outputs)."""
        permutation, _, _ = self._device_values(q.device)
        return layout_ops.reorder_qkv(q, k, v, permutation)

    def restore(self, tensor):
        _, inverse, _ = self._device_values(tensor.device)
        return layout_ops.reorder(tensor, inverse)

    def neighbors(self, device):
        return self._device_values(device)[2]


def build_spatial_layout(grid, block_size=128, max_microtile_tokens=32):
    """Build a reversible Morton-ordered packing with no sequence padding."""
    if grid is None or len(grid) != 3:
        return None
    frames, height, width = (int(value) for value in grid)
    if min(frames, height, width, block_size, max_microtile_tokens) <= 0:
        return None
    tile_h, tile_w = _microtile(height, width, block_size, max_microtile_tokens)
    area = tile_h * tile_w
    tiles_per_block = block_size // area
    rows, cols = height // tile_h, width // tile_w

    # Tile order inside one frame; every frame uses the same order.
    ty, tx = np.meshgrid(np.arange(rows, dtype=np.int64), np.arange(cols, dtype=np.int64),
                         indexing="ij")
    ty, tx = ty.ravel(), tx.ravel()
    order = np.lexsort((tx, ty, _interleave_bits(ty, tx)))
    ty, tx = ty[order], tx[order]
    tiles_per_frame = ty.size

    # Token ids of every tile, tiles in layout order, tokens row-major inside.
    dy, dx = np.meshgrid(np.arange(tile_h), np.arange(tile_w), indexing="ij")
    inner = (dy.ravel()[None] * width + dx.ravel()[None])              # [1, area]
    tile_origin = (ty * tile_h) * width + tx * tile_w                  # [tiles]
    frame_tokens = tile_origin[:, None] + inner                        # [tiles, area]
    frame_offsets = np.arange(frames, dtype=np.int64)[:, None, None] * (height * width)
    permutation = (frame_offsets + frame_tokens[None]).reshape(-1).astype(np.int32)
    inverse = np.empty_like(permutation)
    inverse[permutation] = np.arange(permutation.size, dtype=np.int32)

    # Block of every (frame, tile_y, tile_x); -1 outside the grid.
    tile_index = np.arange(frames * tiles_per_frame)
    frame_of = tile_index // tiles_per_frame
    ty_all = np.tile(ty, frames)
    tx_all = np.tile(tx, frames)
    block_of_tile = np.full((frames, rows, cols), -1, dtype=np.int64)
    block_of_tile[frame_of, ty_all, tx_all] = tile_index // tiles_per_block

    blocks = math.ceil(permutation.size / block_size)
    neighbors = np.full((blocks, 4), -1, dtype=np.int32)
    block_frames = np.full(blocks, -1, dtype=np.int32)
    steps = ((-1, 0), (1, 0), (0, -1), (0, 1))
    for block in range(blocks):
        members = slice(block * tiles_per_block, min((block + 1) * tiles_per_block,
                                                     tile_index.size))
        f, y, x = frame_of[members], ty_all[members], tx_all[members]
        if f.size and (f == f[0]).all():
            block_frames[block] = f[0]
        for direction, (sy, sx) in enumerate(steps):
            ny, nx = y + sy, x + sx
            inside = (ny >= 0) & (ny < rows) & (nx >= 0) & (nx < cols)
            targets = block_of_tile[f[inside], ny[inside], nx[inside]]
            targets = targets[targets != block]
            if targets.size:
                # Most votes; among equal counts the first target seen wins.
                values, first_seen, counts = np.unique(targets, return_index=True,
                                                       return_counts=True)
                winner = np.lexsort((first_seen, -counts))[0]
                neighbors[block, direction] = values[winner]

    return SpatialTokenLayout(
        grid=(frames, height, width),
        block_size=block_size,
        microtile_shape=(tile_h, tile_w),
        permutation_cpu=torch.from_numpy(permutation),
        inverse_cpu=torch.from_numpy(inverse),
        neighbors_cpu=torch.from_numpy(neighbors),
        block_frames_cpu=torch.from_numpy(block_frames),
    )
