"""CPU checks of the end-to-end loop's host pieces: the flow schedule matches
the timesteps the reference's runs recorded, and the RoPE table agrees with the
test-input RoPE restatement."""

import torch

from dit_sparse_atten_amd.wan_dit import WanDiTConfig, flow_timesteps, rope_cos_sin
from tests.golden.inputs import wan_rope_angles


def test_flow_schedule_matches_reference_runs():
    """results/final_flex_hybrid058_update2_release_57k_5step_timing.json:
    timesteps 999, 952, 882, 768, 555."""
    sigmas, timesteps = flow_timesteps(5, 5.0)
    assert timesteps.tolist() == [999.0, 952.0, 882.0, 768.0, 555.0]
    assert sigmas[-1] == 0 and (sigmas[:-1] > sigmas[1:]).all()


def test_rope_table_matches_angles():
    grid = (3, 4, 5)
    table = rope_cos_sin(grid)
    angles = wan_rope_angles(grid)
    assert table.shape == (60, 64, 2)
    torch.testing.assert_close(table[..., 0], torch.cos(angles).float())
    torch.testing.assert_close(table[..., 1], torch.sin(angles).float())


def test_config_is_wan_1_3b_shape():
    c = WanDiTConfig()
    assert (c.layers, c.dim, c.heads, c.head_dim, c.ffn_dim) == (30, 1536, 12, 128, 8960)
