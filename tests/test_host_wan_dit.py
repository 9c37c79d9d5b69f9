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


def test_local_attention_knobs_share_qk_bias_and_scale_norms():
    """qk_position_bias ties one bias vector to every block's q and k
    projections; qk_norm_scale multiplies the q/k RMSNorm weights."""
    from dit_sparse_atten_amd.wan_dit import WanDiT
    small = dict(layers=2, dim=64, heads=1, ffn_dim=64, text_dim=32, freq_dim=16)
    plain = WanDiT(WanDiTConfig(**small), device="cpu", seed=3)
    local = WanDiT(WanDiTConfig(**small, qk_position_bias=1.0, qk_norm_scale=2.0),
                   device="cpu", seed=3)
    for blk_plain, blk in zip(plain.blocks, local.blocks):
        assert blk["q"][1] is blk["k"][1]
        assert not torch.equal(blk_plain["q"][1], blk_plain["k"][1])
        torch.testing.assert_close(blk["norm_q"].abs().mean() / blk_plain["norm_q"].abs().mean(),
                                   torch.tensor(2.0), rtol=0.1, atol=0)
    assert not torch.equal(local.blocks[0]["q"][1], local.blocks[1]["q"][1])
