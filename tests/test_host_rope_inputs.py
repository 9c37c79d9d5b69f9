"""CPU checks of the 3D RoPE used to build BASELINE config 1 inputs: it is a
rotation (norms kept), identity at the origin, and its dot products depend
only on the relative position along each axis."""

import torch

from tests.golden.inputs import apply_rope, wan_rope_angles


def test_split_and_shapes():
    angles = wan_rope_angles((2, 3, 4))
    assert angles.shape == (24, 64)
    # 44 / 42 / 42 head dims -> 22 / 21 / 21 rotation pairs.
    frame_only = wan_rope_angles((2, 1, 1))
    assert (frame_only[1, :22] != 0).all() and (frame_only[1, 22:] == 0).all()


def test_rotation_keeps_norms_and_origin():
    x = torch.randn(1, 24, 2, 128, dtype=torch.float64)
    angles = wan_rope_angles((2, 3, 4))
    y = apply_rope(x, angles)
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1))
    torch.testing.assert_close(y[:, 0], x[:, 0])


def test_relative_position_property():
    grid = (3, 4, 5)
    angles = wan_rope_angles(grid)
    q = torch.randn(1, 1, 1, 128, dtype=torch.float64).expand(1, 60, 1, 128)
    k = torch.randn(1, 1, 1, 128, dtype=torch.float64).expand(1, 60, 1, 128)
    rq, rk = apply_rope(q, angles), apply_rope(k, angles)

    def index(f, y, x):
        return (f * 4 + y) * 5 + x

    a = (rq[0, index(1, 1, 1), 0] * rk[0, index(0, 0, 0), 0]).sum()
    b = (rq[0, index(2, 3, 4), 0] * rk[0, index(1, 2, 3), 0]).sum()
    torch.testing.assert_close(a, b)
