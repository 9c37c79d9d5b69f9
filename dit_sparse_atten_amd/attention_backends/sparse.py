"""Matrix-tile sparse backend (``sparse``) on the libdsa HIP kernels.

Mirrors attention_backends/sparse.py of the reference:
  SparseConfig                      sparse.py:23-48
  exact spatial tile choice         sparse.py:106-138   (_divisors, _spatial_layout)
  tile-major reorder / restore      sparse.py:81-103    -> dsa_permute_rows
  dense bootstrap route             sparse.py:184-233   -> dsa_bsa_fwd (+ LSE),
                                                           dsa_tile_stats, dsa_route_select
  next-step expansion               sparse.py:350-373   -> dsa_expand_route
  sparse attention + statistics     sparse.py:670-751   -> dsa_bsa_fwd (tile blocks),
                                                           dsa_tile_stats (CSR)
  low-mass drop + sink              sparse.py:327-348, 883-884 -> dsa_drop_low_mass
  MatrixSparseBackend               sparse.py:754-942   (same state keys, phases,
                                                         JSONL statistics, probe)
The route state (mask, fp16 mass and centroids) stays on the device; the
reference keeps it on the host and prefetches the next mask to the device, so
``prefetch_route`` is accepted and has nothing to overlap here.
"""

from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass

import numpy as np
import torch

from .. import ops
from .context import routing_context
from .dense import DenseBackend, install


@dataclass(frozen=True)
class SparseConfig:
    """Routing and chunking controls for the matrix-tile backend."""

    # Target tokens per spatial tile; the H x W shape is chosen from exact
    # divisors of the latent grid, so tiles never need padding.
    tile: int = 64
    # Select enough key tiles to reach mass_target, but never more than keep.
    keep: float = 0.625
    mass_target: float = 0.90
    # Accepted for signature compatibility: the kernels walk whole tiles.
    query_chunk: int = 256
    # reuse: previous mask; directional: one-step Q/K moves along the tile
    # centroids; all: the eight coupled Q/K spatial neighbours.
    policy: str = "reuse"
    centroid_threshold: float = 0.15
    # Routes drop blocks below this fraction of the head's mean selected
    # mass, keeping at least one key tile per query tile.
    drop_factor: float = 0.1
    huge_factor: float = 2.0
    # Accepted for signature compatibility (the statistics are fused kernels).
    use_triton: bool = False
    prefetch_route: bool = True
    first_frame_sink: bool = True
    first_layer_dense: bool = True


def _divisors(value):
    small = [d for d in range(1, math.isqrt(value) + 1) if value % d == 0]
    return small + [value // d for d in reversed(small) if d * d != value]


class _SpatialTileLayout:
    """An exact per-frame partition of the (F, H, W) token grid into tiles,
    with the tile-major permutation cached per device."""

    def __init__(self, frames, height, width, tile_h, tile_w):
        self.frames, self.height, self.width = frames, height, width
        self.tile_h, self.tile_w = tile_h, tile_w
        self._device_values = {}

    @property
    def tokens(self):
        return self.frames * self.height * self.width

    @property
    def tile_tokens(self):
        return self.tile_h * self.tile_w

    @property
    def tile_count(self):
        return self.tokens // self.tile_tokens

    @property
    def block_h(self):
        return self.height // self.tile_h

    @property
    def block_w(self):
        return self.width // self.tile_w

    @property
    def signature(self):
        return (self.frames, self.height, self.width, self.tile_h, self.tile_w)

    def permutation(self, device):
        """(tile-major position -> original token, inverse) as device int32."""
        if device not in self._device_values:
            original = np.arange(self.tokens, dtype=np.int32).reshape(
                self.frames, self.block_h, self.tile_h, self.block_w, self.tile_w)
            forward = original.transpose(0, 1, 3, 2, 4).reshape(-1)
            inverse = np.empty_like(forward)
            inverse[forward] = np.arange(self.tokens, dtype=np.int32)
            self._device_values[device] = tuple(
                torch.from_numpy(x).to(device) for x in (forward, inverse))
        return self._device_values[device]

    def to_tile_major(self, *tensors):
        forward, _ = self.permutation(tensors[0].device)
        return ops.permute_tokens(tensors, forward)

    def from_tile_major(self, tensor):
        _, inverse = self.permutation(tensor.device)
        return ops.permute_tokens((tensor,), inverse)[0]


def _spatial_layout(grid, target_tile_tokens, tokens):
    """Choose a near-target spatial tile whose sides exactly divide H and W:
    minimise |log(area / target)| + 0.25 |log(w / h)|, then the area distance,
    then prefer the larger tile (sparse.py:113-138)."""
    if grid is None or len(grid) != 3 or target_tile_tokens <= 0:
        return None
    frames, height, width = (int(value) for value in grid)
    if frames * height * width != tokens:
        return None
    candidates = [(th, tw) for th in _divisors(height) for tw in _divisors(width)]
    tile_h, tile_w = min(candidates, key=lambda shape: (
        abs(math.log(shape[0] * shape[1] / target_tile_tokens))
        + 0.25 * abs(math.log(shape[1] / shape[0])),
        abs(shape[0] * shape[1] - target_tile_tokens),
        -shape[0] * shape[1],
    ))
    return _SpatialTileLayout(frames, height, width, tile_h, tile_w)


class MatrixSparseBackend:
    """Reuse the previous denoising step's matrix-tile route for self-attention."""

    name = "sparse"

    def __init__(self, config=None):
        self.config = config or SparseConfig()
        self.dense = DenseBackend()
        self.state = {}
        self._layouts = {}

    @staticmethod
    def _record_stats(payload):
        """Append opt-in route statistics as JSONL (WAN_SPARSE_STATS_PATH)."""
        path = os.getenv("WAN_SPARSE_STATS_PATH")
        if not path:
            return
        with open(path, "a", encoding="utf-8") as handle:
            handle.write(json.dumps(payload, sort_keys=True) + "\n")

    def _layout(self, grid, tokens):
        key = (tuple(grid) if grid is not None else None, self.config.tile, tokens)
        if key not in self._layouts:
            layout = _spatial_layout(grid, self.config.tile, tokens)
            if layout is not None and (layout.tile_tokens > 128 or layout.tile_count > 16384):
                layout = None  # beyond the kernels' tile limits: dense
            self._layouts[key] = layout
        return self._layouts[key]

    def _expand(self, previous, layout):
        """Any policy other than "reuse" and "all" expands directionally, as
        the reference's `_expand` does."""
        policy = self.config.policy
        if policy == "reuse":
            return previous["mask"]
        if policy != "all":
            policy = "directional"
        return ops.expand_route(
            previous["mask"], (layout.frames, layout.block_h, layout.block_w), policy,
            mass=previous["mass"],
            centroids=[previous[f"centroid_{n}"] for n in ("q_y", "q_x", "k_y", "k_x")],
            centroid_threshold=self.config.centroid_threshold,
            huge_factor=self.config.huge_factor)

    def _sparse_attention(self, q, k, v, scale, layout, deterministic=False):
        c = self.config
        # The reference computes in the input dtype (sparse.py:700-708); so do
        # the kernels: bfloat16, float16, or float32 on the fp32 kernel.
        ops.dtype_code(q.dtype, attention=True)
        output_dtype = q.dtype
        k, v = k.to(q.dtype), v.to(q.dtype)
        # Jointly permuting Q/K/V is attention-equivalent; it only changes
        # which tokens form a tile.
        q, k, v = layout.to_tile_major(q, k, v)
        tokens, heads, head_dim = q.shape[1:]
        if scale is None:
            scale = head_dim ** -0.5
        attention_id, step, branch, _ = routing_context(include_grid=True)
        key = (attention_id, branch, heads, layout.signature)
        tile_shape = (layout.tile_h, layout.tile_w)
        sink = layout.block_h * layout.block_w if c.first_frame_sink else 0
        if step == 0 or key not in self.state:
            # The first observation is dense; its statistics give the exact
            # route (_dense_route, sparse.py:184-233).
            output, _, stats = ops.bsa_fwd_tile_stats(q, k, v, None, tile_shape, scale=scale)
            mask, _ = ops.route_select(stats["mass"], c.mass_target, c.keep, sink_blocks=sink)
            route = {"mask": mask, "mass": stats["mass_f16"], "tile": layout.tile_tokens,
                     "grid": (layout.frames, layout.height, layout.width),
                     "spatial_tile": tile_shape}
            for name in ("q_y", "q_x", "k_y", "k_x"):
                route[f"centroid_{name}"] = stats[f"centroid_{name}"]
            self.state[key] = route
            if os.getenv("WAN_SPARSE_STATS_PATH"):
                self._record_stats({
                    "step": int(step), "attention_id": int(attention_id),
                    "branch": int(branch), "phase": "dense_bootstrap",
                    "tile_count": int(mask.shape[-1]),
                    "executed_tile_fraction": 1.0,
                    "route_mass_fraction": float(
                        (route["mass"].float() * mask).sum().item() / max(1, heads)),
                    "next_tile_fraction": float(mask.float().mean().item()),
                })
            return layout.from_tile_major(output).to(output_dtype)

        previous = self.state[key]
        route = self._expand(previous, layout)
        csr = ops.route_to_csr(route, block_size=layout.tile_tokens)
        collect = c.policy != "reuse"
        if collect:
            # Attention and the statistics of the same softmax in one call
            # (sparse_chunk, sparse.py:670-751).
            output, _, stats = ops.bsa_fwd_tile_stats(q, k, v, csr, tile_shape, scale=scale,
                                                      deterministic=deterministic)
            next_mask, _ = ops.drop_low_mass(route, stats["mass"], c.drop_factor, sink)
            next_state = {"mass": stats["mass_f16"]}
            for name in ("q_y", "q_x", "k_y", "k_x"):
                next_state[f"centroid_{name}"] = stats[f"centroid_{name}"]
        else:
            output = ops.bsa_fwd(q, k, v, csr, scale=scale, block_size=layout.tile_tokens,
                                 deterministic=deterministic)
            # Reuse drops against the stored (fp16) route mass and keeps it.
            next_mask, _ = ops.drop_low_mass(route, previous["mass"], c.drop_factor, sink)
            next_state = {name: previous[name] for name in (
                "mass", "centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x")}
        next_state.update({"mask": next_mask, "tile": layout.tile_tokens,
                           "grid": (layout.frames, layout.height, layout.width),
                           "spatial_tile": tile_shape})
        if os.getenv("WAN_SPARSE_STATS_PATH"):
            self._record_step_stats(previous, route, next_mask, q, k, v, scale, layout,
                                    step, attention_id, branch, heads)
        self.state[key] = next_state
        return layout.from_tile_major(output).to(output_dtype)

    def _record_step_stats(self, previous, route, next_mask, q, k, v, scale, layout, step,
                           attention_id, branch, heads):
        previous_mass = previous["mass"].float()
        route_mass = (previous_mass * route).sum().item() / max(1, heads)
        next_mass = (previous_mass * next_mask).sum().item() / max(1, heads)
        probe = None
        if os.getenv("WAN_DENSE_MASS_PROBE", "0") == "1":
            # Opt-in measurement only: exact dense mass of this step.
            _, lse = ops.bsa_fwd(q, k, v, scale=scale, return_lse=True)
            probe = ops.tile_stats(q, k, lse, (layout.tile_h, layout.tile_w), scale=scale,
                                   centroids=False)["mass"]
            route_mass = (probe * route).sum().item() / max(1, heads)
            next_mass = (probe * next_mask).sum().item() / max(1, heads)
        self._record_stats({
            "step": int(step), "attention_id": int(attention_id), "branch": int(branch),
            "phase": "sparse", "tile_count": int(route.shape[-1]),
            "executed_tile_fraction": float(route.float().mean().item()),
            "route_mass_fraction": float(route_mass) if probe is not None else None,
            "previous_route_mass_estimate": float(route_mass),
            "next_tile_fraction": float(next_mask.float().mean().item()),
            "next_route_mass_fraction": float(next_mass) if probe is not None else None,
            "next_previous_mass_estimate": float(next_mass),
            "mass_semantics": ("same-step dense shadow probe" if probe is not None
                               else "unavailable without WAN_DENSE_MASS_PROBE=1"),
            "drop_factor": float(self.config.drop_factor),
        })

    def __call__(self, q, k, v, softmax_scale=None, **kwargs):
        # The tile statistics take head dims up to 256 (136..256 on the
        # fp32-compute kernel); wider heads run dense.
        if q.shape[1] == k.shape[1] and q.shape[0] == 1 and q.shape[-1] <= 2 * ops.HEAD_DIM:
            attention_id, _, _, grid = routing_context(include_grid=True)
            if self.config.first_layer_dense and attention_id == 0:
                return self.dense(q, k, v, softmax_scale=softmax_scale, **kwargs)
            layout = self._layout(grid, q.shape[1])
            if layout is not None:
                return self._sparse_attention(q, k, v, softmax_scale, layout,
                                              bool(kwargs.get("deterministic", False)))
        return self.dense(q, k, v, softmax_scale=softmax_scale, **kwargs)


def install_sparse(config=None):
    return install(MatrixSparseBackend(config))
