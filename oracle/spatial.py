"""CPU restatement of the token layouts (test infrastructure only).

Follows
  attention_backends/spatial.py:14-183   Morton micro-tile layout of flex_reuse
                                         (_morton_code, _choose_microtile,
                                          build_spatial_layout)
  attention_backends/sparse.py:51-138    exact spatial tile layout of the
                                         matrix-sparse path (_SpatialTileLayout,
                                          _divisors, _spatial_layout)
Written as plain Python loops over the grid, directly from the definitions.
"""

from __future__ import annotations

import math
from collections import Counter, defaultdict

import numpy as np


def morton_code(y, x):
    """Interleave bits: x in even positions, y in odd positions (spatial.py:19-27)."""
    code = 0
    bit = 0
    while (1 << bit) <= max(y, x):
        code |= ((x >> bit) & 1) << (2 * bit)
        code |= ((y >> bit) & 1) << (2 * bit + 1)
        bit += 1
    return code


def choose_microtile(height, width, block_size, max_tokens):
    """Largest exact tile (area <= max_tokens, area | block_size), then least
    elongated (spatial.py:30-43)."""
    best = None
    for tile_h in range(1, height + 1):
        if height % tile_h:
            continue
        for tile_w in range(1, width + 1):
            if width % tile_w:
                continue
            area = tile_h * tile_w
            if area > max_tokens or block_size % area:
                continue
            key = (-area, abs(math.log(tile_w / tile_h)))
            if best is None or key < best[0]:
                best = (key, (tile_h, tile_w))
    return (1, 1) if best is None else best[1]


def spatial_layout(grid, block_size=128, max_microtile_tokens=32):
    """Return dict(microtile, permutation, inverse, neighbors, block_frames).

    permutation[t] is the original token placed at position t; inverse is its
    inverse; neighbors[block, dir] (dir = up, down, left, right) is the
    majority-vote neighbouring block or -1 (spatial.py:99-183).
    """
    frames, height, width = (int(value) for value in grid)
    tile_h, tile_w = choose_microtile(height, width, block_size, max_microtile_tokens)
    area = tile_h * tile_w
    tiles_per_block = block_size // area
    rows, cols = height // tile_h, width // tile_w
    ordered = []
    for frame in range(frames):
        points = [(ty, tx) for ty in range(rows) for tx in range(cols)]
        points.sort(key=lambda p: (morton_code(p[0], p[1]), p[0], p[1]))
        ordered.extend((frame, ty, tx) for ty, tx in points)
    permutation = []
    for frame, ty, tx in ordered:
        for y in range(ty * tile_h, ty * tile_h + tile_h):
            for x in range(tx * tile_w, tx * tile_w + tile_w):
                permutation.append((frame * height + y) * width + x)
    permutation = np.array(permutation, dtype=np.int32)
    inverse = np.empty_like(permutation)
    inverse[permutation] = np.arange(permutation.size, dtype=np.int32)

    tile_block = {}
    block_tiles = defaultdict(list)
    for index, tile in enumerate(ordered):
        tile_block[tile] = index // tiles_per_block
        block_tiles[index // tiles_per_block].append(tile)
    blocks = -(-permutation.size // block_size)
    neighbors = np.full((blocks, 4), -1, dtype=np.int32)
    block_frames = np.full(blocks, -1, dtype=np.int32)
    for block in range(blocks):
        tiles = block_tiles[block]
        frame_set = {tile[0] for tile in tiles}
        if len(frame_set) == 1:
            block_frames[block] = next(iter(frame_set))
        for direction, (dy, dx) in enumerate(((-1, 0), (1, 0), (0, -1), (0, 1))):
            votes = Counter()
            for frame, ty, tx in tiles:
                target = tile_block.get((frame, ty + dy, tx + dx))
                if target is not None and target != block:
                    votes[target] += 1
            if votes:
                # Counter.most_common keeps first-inserted order among equal counts.
                neighbors[block, direction] = votes.most_common(1)[0][0]
    return {
        "microtile": (tile_h, tile_w),
        "permutation": permutation,
        "inverse": inverse,
        "neighbors": neighbors,
        "block_frames": block_frames,
    }


def divisors(value):
    return [d for d in range(1, value + 1) if value % d == 0]


def sparse_tile_shape(grid, target_tile_tokens, tokens):
    """Tile (tile_h, tile_w) of sparse.py:113-138, or None for no exact layout."""
    if grid is None or len(grid) != 3 or target_tile_tokens <= 0:
        return None
    frames, height, width = (int(value) for value in grid)
    if frames * height * width != tokens:
        return None
    best = None
    for tile_h in divisors(height):
        for tile_w in divisors(width):
            area = tile_h * tile_w
            key = (abs(math.log(area / target_tile_tokens))
                   + 0.25 * abs(math.log(tile_w / tile_h)),
                   abs(area - target_tile_tokens), -area)
            if best is None or key < best[0]:
                best = (key, (tile_h, tile_w))
    return best[1]


def tile_major_permutation(grid, tile_shape):
    """perm[t] = original token at tile-major position t (sparse.py:81-92):
    order (frame, block_y, block_x, y_in_tile, x_in_tile)."""
    frames, height, width = grid
    tile_h, tile_w = tile_shape
    perm = []
    for f in range(frames):
        for by in range(height // tile_h):
            for bx in range(width // tile_w):
                for y in range(tile_h):
                    for x in range(tile_w):
                        perm.append((f * height + by * tile_h + y) * width + bx * tile_w + x)
    return np.array(perm, dtype=np.int32)
