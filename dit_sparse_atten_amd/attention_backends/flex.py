"""Hybrid block-sparse backend with sampled, reusable routes (``flex_reuse``).

Mirrors attention_backends/flex.py of the reference, with FlexAttention and
BlockMask replaced by the libdsa HIP kernels and a CSR route:
  FlexReuseConfig / validation      flex.py:43-80, 407-443
  _top_mass_route                   flex.py:83-94      -> dsa_route_select
  _block_attention_mass             flex.py:96-202     -> dsa_block_mass
  _sampled_block_mass               flex.py:205-251    -> dsa_sampled_mass
  _dense_bootstrap                  flex.py:254-272    -> dsa_bsa_fwd (+ LSE), dsa_block_mass
  _pack_route / _build_block_mask   flex.py:275-355    -> dsa_pack_rows / dsa_route_to_csr
  _flex_output                      flex.py:379-399    -> dsa_bsa_fwd
  FlexReuseBackend state machine    flex.py:402-850    (same phases, keys, dispatch,
                                                        prefetch stream and release)
  directional update / frontier     flex.py:517-534, 544-566 -> routing.py kernels
Step 0 returns dense output with an exact (dense + LSE + block-mass pass) or
sampled route; later steps reuse the route, refresh it exactly or update it
from samples (optionally frontier-directed), or dispatch high-keep routes to
the dense kernel.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from .. import ops
from .context import routing_context
from .dense import DenseBackend, install
from .layout_ops import pack_boolean_rows
from .routing import directional_budget_update
from .spatial import build_spatial_layout


@dataclass(frozen=True)
class FlexReuseConfig:
    block_size: int = 128
    keep: float = 0.625
    mass_target: float = 0.90
    # Kept for signature compatibility; the HIP kernels need no compilation.
    compile_kernel: bool = True
    # 0 keeps the step-0 route static; a positive value refreshes the route
    # from exact dense attention every N steps.
    update_interval: int = 0
    # A positive value updates from sampled Q/K blocks every N steps.
    sampled_update_interval: int = 0
    route_samples: int = 2
    sample_query_block_chunk: int = 16
    route_persistence: float = 0.5
    prefetch_sampled_update: bool = True
    prefetch_sampled_bootstrap: bool = True
    total_steps: int | None = None
    bootstrap_mode: str = "exact"
    # Routes at or above this keep fraction run on the dense kernel; None
    # disables automatic per-layer/branch dispatch.
    dense_route_threshold: float | None = None
    release_after_final_step: bool = True
    spatial_reorder: bool = False
    spatial_microtile_tokens: int = 32
    directional_update: bool = False
    direction_min_ratio: float = 0.0
    direction_candidate_bonus: float = 0.0
    route_budget_scale: float = 1.0
    route_exploration_fraction: float = 0.0
    direction_expand_q: bool = True
    direction_expand_k: bool = True
    direction_expand_joint: bool = True
    # Wan's first latent frame is a globally visible key sink.
    first_frame_sink: bool = True
    # Keep the first transformer layer exact on every denoising pass.
    first_layer_dense: bool = True


def _top_mass_route(mass, target, keep):
    """Select K blocks independently for every (head, query-block) row."""
    route, _ = ops.route_select(mass, target, keep)
    return route


def _block_attention_mass(q, k, lse, block_size, scale=None):
    """Recover exact dense block mass from Q, K and the per-query LSE.

    One HIP pass recomputes QK on the matrix cores, normalises every score
    with the LSE of the dense forward and writes one value per 128x128 block;
    no probability tensor is materialised and no atomics are used.
    """
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("Flex bootstrap supports batch-1 self-attention")
    return ops.block_mass(q, k, lse, block_size, scale)


def _sampled_block_mass(q, k, block_size, samples=2, scale=None, query_block_chunk=16):
    """Estimate block mass from evenly sampled Q/K tokens per block.

    One fused kernel scans every sampled key twice per query tile, so no chunk
    of the sampled score matrix is ever materialised (``query_block_chunk`` is
    accepted for signature compatibility).
    """
    if query_block_chunk <= 0:
        raise ValueError("sample_query_block_chunk must be positive")
    return ops.sampled_block_mass(q, k, block_size, samples, scale)


def _dense_with_block_mass(q, k, v, block_size, scale=None):
    """Dense output and its exact block mass (flex.py:254-272 then 158-202),
    in one attention launch for 128-token blocks."""
    if block_size == 128 and q.shape[0] == 1 and q.shape[1] == k.shape[1]:
        output, _, mass = ops.bsa_fwd_block_mass(q, k, v, scale=scale)
        return output, mass
    output, lse = ops.bsa_fwd(q, k, v, scale=scale, return_lse=True)
    return output, _block_attention_mass(q, k, lse, block_size, scale=scale)


def _dense_bootstrap(q, k, v, block_size, mass_target, keep, compile_kernel, scale=None):
    """Return exact dense output and its block-quantized top-mass route."""
    del compile_kernel
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("Flex bootstrap supports batch-1 self-attention")
    output, mass = _dense_with_block_mass(q, k, v, block_size, scale)
    return output, _top_mass_route(mass, mass_target, keep)


def _pack_route(route):
    """Pack a boolean [H,Q,K] route into counts and compact K indices."""
    counts, indices = pack_boolean_rows(route)
    return counts.unsqueeze(0), indices.unsqueeze(0)


def _build_block_mask(route, tokens, block_size, counts=None):
    """Convert a [H,Q,K] route to the CSR the attention kernel walks."""
    if route.ndim != 3 or route.shape[-2] != route.shape[-1]:
        raise ValueError("route must have shape [head, Q-block, K-block]")
    if math.ceil(tokens / block_size) != route.shape[-1]:
        raise ValueError("route does not match the token count")
    return ops.route_to_csr(route, counts, block_size=block_size)


def _flex_output(q, k, v, block_mask, block_size, compile_kernel=True, scale=None,
                 deterministic=False):
    """Block-sparse attention of [B, T, H, D] tensors over a CSR route.

    Partial last blocks are masked inside the kernel, so no padding copies are
    made; the output is contiguous [B, T, H, D].  ``deterministic`` (the
    backend call's own flag) asks for results reproducible bit for bit.
    """
    del compile_kernel
    return ops.bsa_fwd(q, k, v, block_mask, scale=scale, block_size=block_size,
                       deterministic=deterministic)


def _route_keep(block_mask):
    """route.float().mean() from the CSR's device nnz (one 8-byte read)."""
    total = block_mask.route_batches * block_mask.heads * block_mask.q_blocks * block_mask.k_blocks
    return float(np.float32(block_mask.nnz_value()) / np.float32(total))


class FlexReuseBackend:
    """Dense bootstrap followed by reuse with optional exact or sampled route refresh."""

    name = "flex_reuse"

    def __init__(self, config=None):
        self.config = config or FlexReuseConfig()
        c = self.config
        if c.block_size != 128:
            raise ValueError(
                "The minimal flex_reuse backend currently supports only 128-token blocks")
        if c.update_interval < 0:
            raise ValueError("update_interval must be zero or a positive integer")
        if c.sampled_update_interval < 0:
            raise ValueError("sampled_update_interval must be zero or a positive integer")
        if c.update_interval and c.sampled_update_interval:
            raise ValueError("exact and sampled route updates are mutually exclusive")
        if not 0 < c.route_samples <= c.block_size:
            raise ValueError("route_samples must be in [1, block_size]")
        if c.route_persistence < 0:
            raise ValueError("route_persistence must be non-negative")
        if c.bootstrap_mode not in ("exact", "sampled"):
            raise ValueError("bootstrap_mode must be 'exact' or 'sampled'")
        if c.dense_route_threshold is not None and not 0 < c.dense_route_threshold <= 1:
            raise ValueError("dense_route_threshold must be in (0, 1]")
        if not 0 < c.keep <= 1:
            raise ValueError("keep must be in (0, 1]")
        if not 0 < c.mass_target <= 1:
            raise ValueError("mass_target must be in (0, 1]")
        if c.spatial_microtile_tokens <= 0:
            raise ValueError("spatial_microtile_tokens must be positive")
        if c.direction_min_ratio < 0:
            raise ValueError("direction_min_ratio must be non-negative")
        if c.direction_candidate_bonus < 0:
            raise ValueError("direction_candidate_bonus must be non-negative")
        if c.route_budget_scale <= 0:
            raise ValueError("route_budget_scale must be positive")
        if not 0 <= c.route_exploration_fraction <= 1:
            raise ValueError("route_exploration_fraction must be in [0, 1]")
        if c.directional_update and not c.spatial_reorder:
            raise ValueError("directional_update requires spatial_reorder")
        self.dense = DenseBackend()
        self.state = {}
        self.route_streams = {}
        self.spatial_layouts = {}
        self.phase_counts = {
            "dense_bootstrap": 0,
            "sampled_bootstrap": 0,
            "exact_refresh": 0,
            "sampled_update": 0,
            "sparse_reuse": 0,
            "dense_dispatch": 0,
            "first_layer_dense": 0,
        }
        self.finished_routes = []

    # -- route state -----------------------------------------------------

    def _activate_pending_route(self, state):
        pending = state.pop("pending", None)
        if pending is None:
            return
        torch.cuda.current_stream(pending["route"].device).wait_event(pending["ready"])
        state.update({
            "route": pending["route"],
            "frontier": pending.get("frontier"),
            "frontier_count": pending.get("frontier_count"),
            "block_mask": pending["block_mask"],
            "step": pending["source_step"],
        })
        self._update_dispatch(state)

    def _update_dispatch(self, state):
        threshold = self.config.dense_route_threshold
        block_mask = state.get("block_mask")
        keep = (_route_keep(block_mask)
                if state.get("route") is not None and block_mask is not None else None)
        state["keep"] = keep
        frontier = state.get("frontier")
        state["frontier_fraction"] = (
            float(np.float32(state["frontier_count"].item()) / np.float32(frontier.numel()))
            if frontier is not None else None)
        state["dense"] = bool(threshold is not None and keep is not None and keep >= threshold)
        if state["dense"]:
            # A permanently dense state never reads its route again.
            state["route"] = None
            state["block_mask"] = None
            state["frontier"] = None
            state["frontier_count"] = None

    def _is_final_step(self, step):
        return (self.config.release_after_final_step
                and self.config.total_steps is not None
                and step >= self.config.total_steps - 1)

    def _release_route(self, key, state):
        self.finished_routes.append({
            "keep": state.get("keep"),
            "frontier_fraction": state.get("frontier_fraction"),
            "dense": bool(state.get("dense")),
        })
        self.state.pop(key, None)

    def _sink_blocks(self, state):
        grid = state.get("grid")
        if not self.config.first_frame_sink or grid is None:
            return 0
        return math.ceil((grid[1] * grid[2]) / self.config.block_size)

    def _with_frontier(self, state, result):
        """Attach the frontier of the final route when a spatial layout exists."""
        layout = state.get("layout")
        if layout is None:
            result["frontier"] = None
            result["frontier_count"] = None
            return result
        route = result["route"]
        result["frontier"], result["frontier_count"] = ops.frontier_mask(
            route, layout.neighbors(route.device), return_count=True)
        return result

    def _exact_route(self, state, mass):
        """Top-mass route of the exact mass plus the sink (flex.py:708-716, 784-792)."""
        route, counts = ops.route_select(
            mass, self.config.mass_target, self.config.keep,
            sink_blocks=self._sink_blocks(state))
        return self._with_frontier(state, {"route": route, "counts": counts})

    def _sampled_route(self, state, q, k, softmax_scale):
        mass = _sampled_block_mass(
            q, k, self.config.block_size,
            samples=self.config.route_samples,
            scale=softmax_scale,
            query_block_chunk=self.config.sample_query_block_chunk,
        )
        previous = state.get("route")
        layout = state.get("layout")
        if self.config.directional_update and previous is not None and layout is not None:
            c = self.config
            result = directional_budget_update(
                mass, previous, layout.neighbors(q.device), keep=c.keep,
                persistence=c.route_persistence, min_ratio=c.direction_min_ratio,
                candidate_bonus=c.direction_candidate_bonus, budget_scale=c.route_budget_scale,
                exploration_fraction=c.route_exploration_fraction, expand_q=c.direction_expand_q,
                expand_k=c.direction_expand_k, expand_joint=c.direction_expand_joint,
                previous_frontier=state.get("frontier"), sink_blocks=self._sink_blocks(state))
            return self._with_frontier(state, result)
        use_prior = bool(self.config.route_persistence) and previous is not None
        route, counts = ops.route_select(
            mass, self.config.mass_target, self.config.keep,
            previous=previous if use_prior else None,
            persistence=self.config.route_persistence if use_prior else 0.0,
            sink_blocks=self._sink_blocks(state))
        return self._with_frontier(state, {"route": route, "counts": counts})

    def _add_first_frame_sink(self, state, result):
        if not self.config.first_frame_sink:
            return result
        sink = self._sink_blocks(state)
        if not sink:
            return result
        route = result["route"].clone()
        route[..., :sink] = True
        result = dict(result)
        result["route"] = route
        result.pop("counts", None)
        return self._with_frontier(state, result)

    def _install_route(self, state, result, tokens):
        route = result["route"]
        state.update({
            "route": route,
            "frontier": result.get("frontier"),
            "frontier_count": result.get("frontier_count"),
            "block_mask": _build_block_mask(route, tokens, self.config.block_size,
                                            result.get("counts")),
        })

    def _spatial_layout(self, grid, tokens):
        if not self.config.spatial_reorder:
            return None
        if grid is None or math.prod(grid) != tokens:
            return None
        key = (tuple(grid), self.config.block_size, self.config.spatial_microtile_tokens)
        if key not in self.spatial_layouts:
            self.spatial_layouts[key] = build_spatial_layout(
                grid, self.config.block_size, self.config.spatial_microtile_tokens)
        return self.spatial_layouts[key]

    def _prefetch_sampled_route(self, state, q, k, step, softmax_scale,
                                phase="sampled_update"):
        # Default stream priority on purpose.
        stream = self.route_streams.setdefault(q.device, torch.cuda.Stream(device=q.device))
        attention_done = torch.cuda.Event()
        attention_done.record(torch.cuda.current_stream(q.device))
        stream.wait_event(attention_done)
        with torch.cuda.stream(stream):
            q.record_stream(stream)
            k.record_stream(stream)
            result = self._sampled_route(state, q, k, softmax_scale)
            route = result["route"]
            block_mask = _build_block_mask(route, q.shape[1], self.config.block_size,
                                           result.get("counts"))
            ready = torch.cuda.Event()
            ready.record(stream)
        state["pending"] = {
            "route": route,
            "frontier": result.get("frontier"),
            "frontier_count": result.get("frontier_count"),
            "block_mask": block_mask,
            "source_step": step,
            "ready": ready,
        }
        self.phase_counts[phase] += 1

    def profile_summary(self):
        active = [state for state in self.state.values() if state.get("route") is not None]
        keep = [state.get("keep") for state in active] + [
            state["keep"] for state in self.finished_routes if state["keep"] is not None]
        frontier = [state.get("frontier_fraction") for state in active
                    if state.get("frontier_fraction") is not None] + [
            state["frontier_fraction"] for state in self.finished_routes
            if state["frontier_fraction"] is not None]
        return {
            "phase_counts": dict(self.phase_counts),
            "active_routes": len(active),
            "released_routes": len(self.finished_routes),
            "mean_route_keep": sum(keep) / len(keep) if keep else None,
            "mean_frontier_fraction": sum(frontier) / len(frontier) if frontier else None,
            "dense_dispatched_routes": sum(
                bool(state.get("dense")) for state in self.state.values())
            + sum(state["dense"] for state in self.finished_routes),
        }

    # -- call ------------------------------------------------------------

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
        **kwargs,
    ):
        dense_kwargs = dict(q_lens=q_lens, k_lens=k_lens, dropout_p=dropout_p,
                            softmax_scale=softmax_scale, q_scale=q_scale, causal=causal,
                            window_size=window_size, deterministic=deterministic,
                            dtype=dtype, version=version, **kwargs)
        supported = (
            q.shape[0] == 1
            and q.shape[1] == k.shape[1]
            and dropout_p == 0
            and not causal
            and window_size == (-1, -1)
            # The route estimates (sampled and exact block mass) take head
            # dims up to 256; wider heads run dense.
            and q.shape[-1] <= 2 * ops.HEAD_DIM
        )
        if not supported:
            return self.dense(q, k, v, **dense_kwargs)

        attention_id, step, branch, grid = routing_context(include_grid=True)
        if self.config.first_layer_dense and attention_id == 0:
            self.phase_counts["first_layer_dense"] += 1
            return self.dense(q, k, v, **dense_kwargs)
        layout = self._spatial_layout(grid, q.shape[1])
        if self.config.spatial_reorder and layout is None:
            return self.dense(q, k, v, **dense_kwargs)

        key = (attention_id, branch, q.shape[1], q.shape[2], q.shape[3], q.device,
               layout.signature if layout is not None else None)
        state = self.state.get(key) if step != 0 else None
        if state is not None:
            self._activate_pending_route(state)
            if state.get("dense"):
                # Dense attention commutes with the token permutation, so a
                # dense-dispatched state skips the reorder and restore that the
                # reference performs first (flex.py:690-700, 766-775).
                self.phase_counts["dense_dispatch"] += 1
                if self._is_final_step(step):
                    self._release_route(key, state)
                return self.dense(q, k, v, **dense_kwargs)

        output_dtype = q.dtype
        q = q.to(dtype)
        k = k.to(dtype)
        v = v.to(dtype)
        if q_scale is not None:
            q = q * q_scale
        if layout is not None:
            q, k, v = layout.reorder_qkv(q, k, v)

        def finish(output):
            if layout is not None:
                output = layout.restore(output)
            return output.to(output_dtype)

        def dense_output():
            return self.dense(q, k, v, dropout_p=0.0, softmax_scale=softmax_scale,
                              q_scale=None, causal=False, window_size=(-1, -1), dtype=dtype)

        if state is None:
            state = {
                "route": None,
                "frontier": None,
                "block_mask": None,
                "step": step,
                "layout": layout,
                "grid": grid,
            }
            self.state[key] = state
            if self.config.bootstrap_mode == "exact":
                # Dense output with its exact block mass.
                output, mass = _dense_with_block_mass(q, k, v, self.config.block_size,
                                                      softmax_scale)
                self._install_route(state, self._exact_route(state, mass), q.shape[1])
                self._update_dispatch(state)
                self.phase_counts["dense_bootstrap"] += 1
            # Sampled bootstrap: complete dense output, route from samples.
            elif (self.config.prefetch_sampled_bootstrap
                    and (self.config.total_steps is None
                         or step < self.config.total_steps - 1)):
                output = dense_output()
                self._prefetch_sampled_route(state, q, k, step, softmax_scale,
                                             phase="sampled_bootstrap")
            else:
                output = dense_output()
                result = self._sampled_route(state, q, k, softmax_scale)
                self._install_route(state, result, q.shape[1])
                self._update_dispatch(state)
                self.phase_counts["sampled_bootstrap"] += 1
            if self._is_final_step(step):
                self._release_route(key, self.state[key])
            return finish(output)

        if (self.config.update_interval > 0
                and (step - state["step"]) >= self.config.update_interval
                and not self._is_final_step(step)):
            output, mass = _dense_with_block_mass(q, k, v, self.config.block_size,
                                                  softmax_scale)
            state["block_mask"] = None
            self._install_route(state, self._exact_route(state, mass), q.shape[1])
            state["step"] = step
            self._update_dispatch(state)
            self.phase_counts["exact_refresh"] += 1
            return finish(output)

        sampled_update_due = (
            self.config.sampled_update_interval > 0
            and (step - state["step"]) >= self.config.sampled_update_interval
            and (self.config.total_steps is None or step < self.config.total_steps - 1)
        )
        if sampled_update_due and not self.config.prefetch_sampled_update:
            # The old route will not execute this step; drop it before the
            # replacement is built.
            state["block_mask"] = None
            result = self._sampled_route(state, q, k, softmax_scale)
            self._install_route(state, result, q.shape[1])
            state["step"] = step
            self._update_dispatch(state)
            self.phase_counts["sampled_update"] += 1
            if state.get("dense"):
                self.phase_counts["dense_dispatch"] += 1
                return finish(dense_output())

        output = _flex_output(q, k, v, state["block_mask"], self.config.block_size,
                              scale=softmax_scale, deterministic=deterministic)
        self.phase_counts["sparse_reuse"] += 1
        if self.config.prefetch_sampled_update and sampled_update_due:
            state["block_mask"] = None
            self._prefetch_sampled_route(state, q, k, step, softmax_scale)
        if self._is_final_step(step):
            self._release_route(key, state)
        return finish(output)


def install_flex_reuse(config=None):
    return install(FlexReuseBackend(config))
