"""Host-side logic of the backend mirror (CPU): spatial layout builder against
the reference's golden permutation/neighbour tables, config validation and the
routing context bookkeeping."""

import importlib
import sys
import types
from pathlib import Path

import numpy as np
import pytest
import torch

from dit_sparse_atten_amd.attention_backends import context
from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend, FlexReuseConfig
from dit_sparse_atten_amd.attention_backends.spatial import build_spatial_layout

GOLDEN = Path(__file__).resolve().parent / "golden"


def _spatial_cases():
    data = np.load(GOLDEN / "spatial_layout.npz", allow_pickle=False)
    return data, sorted({key.split("__")[0] for key in data.files})


@pytest.mark.parametrize("name", _spatial_cases()[1])
def test_layout_builder_matches_reference_golden(name):
    data, _ = _spatial_cases()
    params = [int(x) for x in data[f"{name}__params"]]
    layout = build_spatial_layout(tuple(params[:3]), params[3], params[4])
    assert layout.microtile_shape == tuple(data[f"{name}__microtile"].tolist())
    assert np.array_equal(layout.permutation_cpu.numpy(), data[f"{name}__permutation"])
    assert np.array_equal(layout.neighbors_cpu.numpy(), data[f"{name}__neighbors"])
    assert np.array_equal(layout.block_frames_cpu.numpy(), data[f"{name}__block_frames"])
    perm, inv = layout.permutation_cpu, layout.inverse_cpu
    assert torch.equal(perm[inv.long()], torch.arange(perm.numel(), dtype=torch.int32))


def test_layout_signature_and_counts():
    layout = build_spatial_layout((16, 45, 80), block_size=128)
    assert layout.microtile_shape == (1, 16)
    assert (layout.tokens, layout.blocks) == (57600, 450)
    assert layout.signature == ((16, 45, 80), 128, (1, 16))
    assert build_spatial_layout(None) is None
    assert build_spatial_layout((0, 4, 4)) is None


def test_flex_config_validation_matches_reference():
    """tests/test_runtime_context.py:63-84 (ValueError list)."""
    for config in (
        FlexReuseConfig(update_interval=-1, bootstrap_mode="sampled"),
        FlexReuseConfig(keep=0, bootstrap_mode="sampled"),
        FlexReuseConfig(mass_target=1.1, bootstrap_mode="sampled"),
        FlexReuseConfig(update_interval=1, sampled_update_interval=1, bootstrap_mode="sampled"),
        FlexReuseConfig(route_samples=129, bootstrap_mode="sampled"),
        FlexReuseConfig(route_persistence=-0.1, bootstrap_mode="sampled"),
        FlexReuseConfig(bootstrap_mode="invalid"),
        FlexReuseConfig(dense_route_threshold=0, bootstrap_mode="sampled"),
        FlexReuseConfig(directional_update=True, spatial_reorder=False, bootstrap_mode="sampled"),
        FlexReuseConfig(route_budget_scale=0, bootstrap_mode="sampled"),
        FlexReuseConfig(block_size=64, bootstrap_mode="sampled"),
    ):
        with pytest.raises(ValueError):
            FlexReuseBackend(config)
    assert FlexReuseConfig().update_interval == 0


def test_flex_sink_known_answer():
    """tests/test_flex_route_update.py:106-112."""
    backend = FlexReuseBackend(FlexReuseConfig(bootstrap_mode="sampled"))
    route = torch.zeros(2, 4, 4, dtype=torch.bool)
    result = backend._add_first_frame_sink({"grid": (2, 8, 16), "layout": None},
                                           {"route": route})
    assert result["route"][..., 0].all()
    assert not result["route"][..., 1:].any()


def _fake_wan(monkeypatch):
    """Fake wan.modules.* as in the reference's tests/test_runtime_context.py:8-38."""
    wan = types.ModuleType("wan")
    modules = types.ModuleType("wan.modules")
    model = types.ModuleType("wan.modules.model")
    attention = types.ModuleType("wan.modules.attention")

    class WanSelfAttention:
        def __init__(self):
            pass

        def forward(self, x, seq_lens, grid_sizes, freqs):
            return x

    class WanModel:
        def parameters(self):
            return iter(())

        def forward(self, x, t, **kwargs):
            return x

    model.WanSelfAttention = WanSelfAttention
    model.WanModel = WanModel
    wan.modules = modules
    modules.model = model
    modules.attention = attention
    for name, module in (("wan", wan), ("wan.modules", modules),
                         ("wan.modules.model", model), ("wan.modules.attention", attention)):
        monkeypatch.setitem(sys.modules, name, module)
    return model


def test_runtime_context_injects_step_branch_layer_and_grid(monkeypatch):
    """tests/test_runtime_context.py:41-60."""
    model_module = _fake_wan(monkeypatch)
    context.install_wan_context()
    model = model_module.WanModel()
    attention = model_module.WanSelfAttention()
    model.forward(torch.ones(()), torch.tensor([10.0]))
    attention.forward(torch.ones(()), None, torch.tensor([[2, 3, 4]]), None)
    assert context.routing_context(include_grid=True) == (0, 0, 0, (2, 3, 4))
    model.forward(torch.ones(()), torch.tensor([10.0]))
    assert context.routing_context()[1:] == (0, 1)
    model.forward(torch.ones(()), torch.tensor([9.0]))
    assert context.routing_context()[1:] == (1, 0)
    profile = context.runtime_profile()
    assert profile["denoising_steps_observed"] == 2
    assert profile["model_forward_calls"] == 3
    context.reset_runtime_state()


def test_product_path_rejects_cpu_tensors():
    """No CPU fallback: the kernels refuse host tensors loudly."""
    from dit_sparse_atten_amd.attention_backends import DenseBackend
    q = torch.randn(1, 8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        DenseBackend()(q, q, q)
