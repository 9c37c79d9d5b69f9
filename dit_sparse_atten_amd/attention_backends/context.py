"""Runtime routing context: layer, denoising step, CFG branch and token grid.

Mirrors attention_backends/context.py of the reference: the backends read
``routing_context()`` (context.py:43-49) to key their routes; model
integrations set the fields before every attention call.  ``install_wan_context``
injects the same bookkeeping into an importable Wan checkout
(context.py:79-156), and ``runtime_profile`` reports per-forward device time
(context.py:236-259).
"""

from __future__ import annotations

import functools
import math
import time
from dataclasses import dataclass, field

import torch


@dataclass
class _RuntimeState:
    attention_id: int = -1
    denoising_step: int = -1
    cfg_branch: int = -1
    grid_size: tuple[int, int, int] | None = None
    last_timestep: float | None = None
    forward_calls: list[dict] = field(default_factory=list)


_STATE = _RuntimeState()


def reset_runtime_state():
    """Reset per-generation routing and timing state."""
    global _STATE
    _STATE = _RuntimeState()


def routing_context(include_grid=False):
    """(attention_id, denoising_step, cfg_branch[, grid]) of the current call."""
    values = (_STATE.attention_id, _STATE.denoising_step, _STATE.cfg_branch)
    return values + (_STATE.grid_size,) if include_grid else values


def set_routing_context(attention_id=None, step=None, branch=None, grid=None):
    """Set any of the context fields (harnesses and model integrations)."""
    if attention_id is not None:
        _STATE.attention_id = int(attention_id)
    if step is not None:
        _STATE.denoising_step = int(step)
    if branch is not None:
        _STATE.cfg_branch = int(branch)
    if grid is not None:
        _STATE.grid_size = tuple(int(value) for value in grid)


def _timestep_value(args, kwargs):
    timestep = kwargs.get("t", args[1] if len(args) > 1 else None)
    if timestep is None:
        return None
    if torch.is_tensor(timestep):
        return float(timestep.detach().flatten()[0].item())
    return float(timestep)


def _grid_value(args, kwargs):
    grid_sizes = kwargs.get("grid_sizes", args[2] if len(args) > 2 else None)
    if grid_sizes is None:
        return None
    grid = grid_sizes[0]
    if torch.is_tensor(grid):
        grid = grid.detach().cpu().tolist()
    return tuple(int(value) for value in grid)


def observe_model_forward(timestep):
    """Advance step/branch bookkeeping for one model forward.

    A new timestep starts a denoising step with branch 0; a repeated timestep
    is the next CFG branch (context.py:117-125).
    """
    if timestep is None:
        return
    if _STATE.last_timestep is None or not math.isclose(timestep, _STATE.last_timestep):
        _STATE.denoising_step += 1
        _STATE.cfg_branch = 0
        _STATE.last_timestep = timestep
    else:
        _STATE.cfg_branch += 1


def timed_call(function, *args, timestep=None, device=None, **kwargs):
    """Run one model forward with step/branch bookkeeping and device events."""
    observe_model_forward(timestep)
    start_event = end_event = None
    if device is not None and torch.device(device).type == "cuda":
        start_event = torch.cuda.Event(enable_timing=True)
        end_event = torch.cuda.Event(enable_timing=True)
        start_event.record()
    wall_started = time.perf_counter()
    try:
        return function(*args, **kwargs)
    finally:
        if end_event is not None:
            end_event.record()
        _STATE.forward_calls.append({
            "step": _STATE.denoising_step,
            "branch": _STATE.cfg_branch,
            "timestep": timestep,
            "wall_seconds_unsynchronized": time.perf_counter() - wall_started,
            "start_event": start_event,
            "end_event": end_event,
        })


def install_wan_context():
    """Inject routing context into an imported Wan model (``wan.modules.model``).

    Idempotent; must run before model construction so that every
    self-attention module receives a stable ID.
    """
    import wan.modules.model as model_module

    if getattr(model_module, "_DSA_CONTEXT_INSTALLED", False):
        return
    reset_runtime_state()
    next_id = [0]
    attention_cls = model_module.WanSelfAttention
    model_cls = model_module.WanModel
    original_init = attention_cls.__init__
    original_forward = attention_cls.forward
    original_model_forward = model_cls.forward

    @functools.wraps(original_init)
    def attention_init(instance, *args, **kwargs):
        original_init(instance, *args, **kwargs)
        instance._dsa_attention_id = next_id[0]
        next_id[0] += 1

    @functools.wraps(original_forward)
    def attention_forward(instance, *args, **kwargs):
        _STATE.attention_id = instance._dsa_attention_id
        grid = _grid_value(args, kwargs)
        if grid is not None:
            _STATE.grid_size = grid
        return original_forward(instance, *args, **kwargs)

    @functools.wraps(original_model_forward)
    def model_forward(instance, *args, **kwargs):
        try:
            device = next(instance.parameters()).device
        except (AttributeError, StopIteration):
            device = None
        return timed_call(original_model_forward, instance, *args,
                          timestep=_timestep_value(args, kwargs), device=device, **kwargs)

    attention_cls.__init__ = attention_init
    attention_cls.forward = attention_forward
    model_cls.forward = model_forward
    model_module._DSA_CONTEXT_INSTALLED = True


def runtime_profile():
    """Synchronize recorded events and return serializable per-forward timing."""
    if any(call["end_event"] is not None for call in _STATE.forward_calls):
        torch.cuda.synchronize()
    calls = []
    for call in _STATE.forward_calls:
        elapsed = None
        if call["start_event"] is not None:
            elapsed = call["start_event"].elapsed_time(call["end_event"]) / 1000
        calls.append({
            "step": call["step"],
            "branch": call["branch"],
            "timestep": call["timestep"],
            "cuda_seconds": elapsed,
            "wall_seconds_unsynchronized": call["wall_seconds_unsynchronized"],
        })
    device_seconds = [call["cuda_seconds"] for call in calls if call["cuda_seconds"] is not None]
    return {
        "denoising_steps_observed": len({call["step"] for call in calls}),
        "model_forward_calls": len(calls),
        "model_forward_cuda_seconds": sum(device_seconds) if device_seconds else None,
        "calls": calls,
    }
