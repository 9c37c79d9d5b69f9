"""GPU parity of the route-update and layout kernels against the oracle and the
reference's golden vectors.  Routes, CSR, packing and gathers are bit-exact."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import route as R
from oracle import spatial as S
from tests.golden.inputs import clustered_qkv

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


@pytest.mark.parametrize("case", ["bf16_s16", "bf16_partial_s16", "f16_partial_s16",
                                  "bf16_partial_s12", "bf16_partial_s48"])
def test_sampled_mass_matches_reference_golden(ops, cuda_device, case):
    """The reference's own _sampled_block_mass outputs: bf16 and fp16 inputs
    (scores rounded in the input type), partial last blocks, 16, 12 and 48
    samples per block."""
    from tests.test_oracle_route import GOLDEN_DTYPES
    data = _load("sampled_mass")
    tokens, heads, dim, block, samples, code, seed = (int(x) for x in data[f"{case}__params"])
    dtype, score_dtype = GOLDEN_DTYPES[code]
    q, k, _ = clustered_qkv(tokens, heads, dim, group=block, seed=seed, dtype=dtype)
    mass = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, samples)
    torch.cuda.synchronize()
    got = mass.cpu().numpy()
    np.testing.assert_allclose(got, data[f"{case}__mass"], atol=2e-3, rtol=2e-3)
    oracle = R.sampled_block_mass(q.float().numpy(), k.float().numpy(), block, samples,
                                  score_dtype=score_dtype)
    np.testing.assert_allclose(got, oracle, atol=2e-3, rtol=2e-3)
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("samples", [1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 33, 48, 64, 100, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sampled_mass_sample_counts(ops, cuda_device, samples, dtype):
    """Any sample count 1..block (flex.py:219-231 accepts 1..block_size):
    powers of two up to 32 directly, other counts padded to the next power of
    two, 64 and 128 with block sums across waves; partial last block."""
    tokens, heads, block = 1000, 3, 128
    q, k, _ = clustered_qkv(tokens, heads, 128, group=block, seed=samples, dtype=dtype)
    got = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, samples)
    torch.cuda.synchronize()
    oracle = R.sampled_block_mass(q.float().numpy(), k.float().numpy(), block, samples,
                                  score_dtype="bf16" if dtype == torch.bfloat16 else "fp16")
    np.testing.assert_allclose(got.cpu().numpy(), oracle, atol=2e-3, rtol=2e-3)
    np.testing.assert_allclose(got.sum(-1).cpu().numpy(), 1.0, atol=1e-5)
    # Deterministic: block sums have a fixed order, without atomics.
    again = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, samples)
    assert torch.equal(again, got)


@pytest.mark.parametrize("tokens,samples", [(128, 1), (128, 2), (128, 3), (128, 4), (512, 1),
                                            (256, 2), (300, 1)])
def test_sampled_mass_few_sampled_keys(ops, cuda_device, tokens, samples):
    """At most 4 sampled keys in all (blocks * samples <= 4, or a padded
    sample count): lanes whose keys are all masked must contribute zero, not
    NaN, so the mass is finite, rows sum to 1 and match the oracle."""
    block, heads = 128, 2
    q, k, _ = clustered_qkv(tokens, heads, 128, group=block, seed=tokens + samples,
                            dtype=torch.bfloat16)
    got = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, samples)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    assert np.isfinite(got).all()
    oracle = R.sampled_block_mass(q.float().numpy(), k.float().numpy(), block, samples,
                                  score_dtype="bf16")
    np.testing.assert_allclose(got, oracle, atol=2e-3, rtol=2e-3)
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=1e-5)


def test_full_sampling_at_block_128_matches_exact_block_mass(ops, cuda_device):
    """samples == block == 128 (the reference's identity, test_flex_backend.py:
    43-53, at the production block size): mass = exact mass / block, up to
    the bf16 rounding of the scores."""
    tokens, heads, block = 128 * 6, 2, 128
    generator = torch.Generator().manual_seed(6)
    q = torch.randn(1, tokens, heads, 128, generator=generator).to(torch.bfloat16)
    k = torch.randn(1, tokens, heads, 128, generator=generator).to(torch.bfloat16)
    got = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, block)
    torch.cuda.synchronize()
    scores = np.einsum("bqhd,bkhd->bhqk", q.double().numpy(), k.double().numpy()) / math.sqrt(128)
    probabilities = np.exp(scores - scores.max(-1, keepdims=True))
    probabilities /= probabilities.sum(-1, keepdims=True)
    blocks = tokens // block
    exact = probabilities[0].reshape(heads, blocks, block, blocks, block).sum((2, 4))
    np.testing.assert_allclose(got.cpu().numpy(), exact / block, atol=3e-3, rtol=3e-2)


def test_full_sampling_matches_exact_block_mass(ops, cuda_device):
    """samples == block gives exact mass / block (reference test_flex_backend.py:43-53),
    up to the bf16 rounding of scores that a bf16 call applies."""
    tokens, heads, block = 16 * 12, 2, 16
    generator = torch.Generator().manual_seed(4)
    q = torch.randn(1, tokens, heads, 128, generator=generator).to(torch.bfloat16)
    k = torch.randn(1, tokens, heads, 128, generator=generator).to(torch.bfloat16)
    got = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), block, block)
    torch.cuda.synchronize()
    scores = np.einsum("bqhd,bkhd->bhqk", q.double().numpy(), k.double().numpy()) / math.sqrt(128)
    probabilities = np.exp(scores - scores.max(-1, keepdims=True))
    probabilities /= probabilities.sum(-1, keepdims=True)
    blocks = tokens // block
    exact = probabilities[0].reshape(heads, blocks, block, blocks, block).sum((2, 4))
    np.testing.assert_allclose(got.cpu().numpy(), exact / block, atol=3e-3, rtol=3e-2)


def _random_mass(shape, seed, alpha=0.3):
    rng = np.random.default_rng(seed)
    return rng.dirichlet(np.full(shape[-1], alpha), size=shape[:-1]).astype(np.float32)


@pytest.mark.parametrize("prior", [False, True])
def test_route_select_bit_exact_at_config3_shape(ops, cuda_device, prior):
    """40 heads x 450 x 450, target .95, cap ceil(450*.625)=282, 29 sink columns."""
    mass = _random_mass((40, 450, 450), seed=11)
    rng = np.random.default_rng(12)
    previous = rng.random((40, 450, 450)) < 0.625 if prior else None
    route, counts = ops.route_select(
        torch.from_numpy(mass).to(cuda_device), 0.95, 0.625,
        previous=None if previous is None else torch.from_numpy(previous).to(cuda_device),
        persistence=0.5 if prior else 0.0, sink_blocks=29)
    torch.cuda.synchronize()
    expected = R.sampled_route(None, None, 128, 16, 0.95, 0.625, previous=previous, rho=0.5,
                               grid=(16, 45, 80), mass=mass)
    got = route.cpu().numpy()
    assert (got == expected).all(), np.argwhere((got != expected).any(-1))[:5]
    assert (counts.cpu().numpy() == expected.sum(-1)).all()


@pytest.mark.parametrize("case", ["dirichlet", "dirichlet_t90_k50", "ties", "flat_cap",
                                  "known_answer"])
def test_route_select_golden_cases(ops, cuda_device, case):
    data = _load("top_mass_route")
    mass = data[f"{case}__mass"]
    target, keep = data[f"{case}__params"]
    route, _ = ops.route_select(torch.from_numpy(mass).to(cuda_device), target, keep)
    torch.cuda.synchronize()
    got = route.cpu().numpy()
    assert (got == R.top_mass_route(mass, target, keep)).all()
    # Against the reference itself: equal selected-value multisets per row.
    expected = data[f"{case}__route"]
    for row_got, row_exp, row_mass in zip(got.reshape(-1, mass.shape[-1]),
                                          expected.reshape(-1, mass.shape[-1]),
                                          mass.reshape(-1, mass.shape[-1])):
        assert np.array_equal(np.sort(row_mass[row_got]), np.sort(row_mass[row_exp]))


def test_route_select_prior_golden(ops, cuda_device):
    data = _load("sampled_route")
    route, _ = ops.route_select(
        torch.from_numpy(data["mass"]).to(cuda_device), 0.95, 0.625,
        previous=torch.from_numpy(data["previous"]).to(cuda_device), persistence=0.5)
    torch.cuda.synchronize()
    primed = R.persistence_prior(data["mass"], data["previous"], 0.5)
    assert (route.cpu().numpy() == R.top_mass_route(primed, 0.95, 0.625)).all()


def test_route_select_rounding_boundaries(ops, cuda_device):
    """Rows built so that prefix sums fall on and next to fp32 rounding ties."""
    rng = np.random.default_rng(3)
    rows = []
    for _ in range(256):
        base = np.float32(rng.uniform(0.01, 0.2))
        ulp = np.spacing(base)
        row = np.full(64, base, np.float32)
        row[rng.integers(0, 64, 8)] += ulp * rng.integers(-3, 4, 8).astype(np.float32)
        row[rng.integers(0, 64, 4)] = np.float32(2.0 ** -rng.integers(20, 40))
        rows.append(row)
    mass = np.stack(rows).astype(np.float32)
    for target in (0.5, 0.9, 0.95, 1.0):
        route, _ = ops.route_select(torch.from_numpy(mass).to(cuda_device), target, 1.0)
        torch.cuda.synchronize()
        assert (route.cpu().numpy() == R.top_mass_route(mass, target, 1.0)).all(), target


def test_csr_and_pack_bit_exact(ops, cuda_device):
    rng = np.random.default_rng(19)
    route = rng.random((5, 37, 450)) < 0.61  # reference test_flex_backend.py:30-40
    dev = torch.from_numpy(route).to(cuda_device)
    counts, indices = ops.pack_rows(dev)
    csr = ops.route_to_csr(dev)
    torch.cuda.synchronize()
    exp_counts, exp_indices = R.pack_rows(route)
    assert (counts.cpu().numpy() == exp_counts).all()
    assert (indices.cpu().numpy() == exp_indices).all()
    row_ptr, col_idx, _ = R.to_csr(route)
    assert (csr.row_ptr.cpu().numpy() == row_ptr).all()
    nnz = csr.nnz_value()
    assert nnz == route.sum()
    assert (csr.col_idx[:nnz].cpu().numpy() == col_idx).all()
    assert (csr.to_route().cpu().numpy()[0] == route).all() if csr._route is None else True


def test_pack_rows_known_answer(ops, cuda_device):
    route = torch.tensor([[[True, False, True], [False, True, False]],
                          [[False, True, True], [True, False, True]]], device=cuda_device)
    counts, indices = ops.pack_rows(route)
    assert counts.cpu().tolist() == [[2, 1], [2, 2]]
    for head in range(2):
        for query in range(2):
            count = counts[head, query].item()
            assert indices[head, query, :count].cpu().tolist() == \
                torch.where(route[head, query].cpu())[0].tolist()


@pytest.mark.parametrize("grid,head_major", [((16, 45, 80), False), ((2, 4, 8), True),
                                             ((21, 30, 52), True)])
def test_permute_tokens_bit_exact(ops, cuda_device, grid, head_major):
    layout = S.spatial_layout(grid, 8 if grid == (2, 4, 8) else 128)
    tokens = layout["permutation"].size
    heads = 5 if tokens > 10000 else 3
    generator = torch.Generator().manual_seed(1)
    base = [torch.randn(1, heads, tokens, 128, generator=generator).to(torch.bfloat16)
            for _ in range(3)]
    views = [t.to(cuda_device).transpose(1, 2) for t in base]  # BHSD memory, BSHD view
    perm = torch.from_numpy(layout["permutation"]).to(cuda_device)
    out = ops.permute_tokens(views, perm, head_major=head_major)
    inv = torch.from_numpy(layout["inverse"]).to(cuda_device)
    back = ops.permute_tokens(out, inv)
    torch.cuda.synchronize()
    for got, src, restored in zip(out, base, back):
        expected = src.transpose(1, 2)[:, layout["permutation"]]
        assert torch.equal(got.cpu(), expected)
        assert torch.equal(restored.cpu(), src.transpose(1, 2))


@pytest.mark.parametrize("tokens,heads,dim", [(1001, 3, 64), (7, 40, 128), (33, 1, 8)])
def test_permute_tokens_ragged_layouts_and_invalid_indices(ops, cuda_device, tokens, heads, dim):
    """Odd token counts (a last head-major group of one token), 16-byte rows,
    batch 2, a mix of head-major and token-major destinations in one launch,
    and out-of-range indices, whose destination rows stay untouched."""
    generator = torch.Generator().manual_seed(tokens)
    sources = [torch.randn(2, tokens, heads, dim, generator=generator).to(torch.bfloat16)
               for _ in range(3)]
    perm = torch.randperm(tokens, generator=generator).to(torch.int32)
    perm[::5] = -1
    perm[2::7] = tokens + 3
    valid = (perm >= 0) & (perm < tokens)
    for layouts in (("head", "head", "head"), ("token", "token", "token"),
                    ("head", "token", "head")):
        out = []
        for layout in layouts:
            shape = (2, heads, tokens, dim) if layout == "head" else (2, tokens, heads, dim)
            t = torch.full(shape, 7.0, dtype=torch.bfloat16, device=cuda_device)
            out.append(t.transpose(1, 2) if layout == "head" else t)
        ops.permute_tokens([s.to(cuda_device) for s in sources], perm.to(cuda_device), out=out)
        torch.cuda.synchronize()
        for got, src in zip(out, sources):
            expected = torch.full_like(src, 7.0)
            expected[:, valid] = src[:, perm[valid].long()]
            assert torch.equal(got.cpu(), expected), layouts


@pytest.mark.parametrize("keys", [591, 1339, 2048])
def test_route_select_beyond_1024_keys(ops, cuda_device, keys):
    """Longer videos: 81 frames at 720p (591 blocks), 1080p x 81 frames
    (1,339 blocks) and the 2,048-key maximum; prior and sink, bit-exact."""
    mass = _random_mass((2, 24, keys), seed=keys)
    rng = np.random.default_rng(keys + 1)
    previous = rng.random((2, 24, keys)) < 0.625
    route, counts = ops.route_select(
        torch.from_numpy(mass).to(cuda_device), 0.95, 0.625,
        previous=torch.from_numpy(previous).to(cuda_device), persistence=0.5, sink_blocks=29)
    torch.cuda.synchronize()
    expected = R.top_mass_route(R.persistence_prior(mass, previous, 0.5), 0.95, 0.625)
    expected[..., :29] = True
    got = route.cpu().numpy()
    assert (got == expected).all(), np.argwhere((got != expected).any(-1))[:5]
    assert (counts.cpu().numpy() == expected.sum(-1)).all()


@pytest.mark.parametrize("keys", [2049, 3000, 4096, 6000, 16384])
def test_route_select_beyond_2048_keys(ops, cuda_device, keys):
    """Rows of more than 2,048 key blocks (a workgroup per row, LDS sort):
    bit-exact with the oracle, prior and sink included."""
    rows = 8 if keys <= 6000 else 3
    mass = _random_mass((1, rows, keys), seed=keys)
    rng = np.random.default_rng(keys + 1)
    previous = rng.random((1, rows, keys)) < 0.625
    route, counts = ops.route_select(
        torch.from_numpy(mass).to(cuda_device), 0.95, 0.625,
        previous=torch.from_numpy(previous).to(cuda_device), persistence=0.5, sink_blocks=29)
    plain, _ = ops.route_select(torch.from_numpy(mass).to(cuda_device), 0.9, 0.5)
    torch.cuda.synchronize()
    expected = R.top_mass_route(R.persistence_prior(mass, previous, 0.5), 0.95, 0.625)
    expected[..., :29] = True
    got = route.cpu().numpy()
    assert (got == expected).all(), np.argwhere((got != expected).any(-1))[:5]
    assert (counts.cpu().numpy() == expected.sum(-1)).all()
    assert (plain.cpu().numpy() == R.top_mass_route(mass, 0.9, 0.5)).all()


@pytest.mark.parametrize("keys", [450, 3000])
def test_route_select_any_magnitude(ops, cuda_device, keys):
    """Power-of-two scales of the mass (row sums from about 2^-90 to 2^40,
    far past the 2^11 a fixed 2^52 fixed point holds) give the unscaled
    route, and the oracle's, bit for bit."""
    mass = _random_mass((2, 16, keys), seed=keys + 7)
    rng = np.random.default_rng(keys + 8)
    previous = rng.random(mass.shape) < 0.6
    base = R.top_mass_route(R.persistence_prior(mass, previous, 0.5), 0.95, 0.625)
    for exponent in (-90, 0, 40):
        scaled = np.ldexp(mass, exponent).astype(np.float32)
        route, _ = ops.route_select(
            torch.from_numpy(scaled).to(cuda_device), 0.95, 0.625,
            previous=torch.from_numpy(previous).to(cuda_device), persistence=0.5)
        torch.cuda.synchronize()
        assert (route.cpu().numpy() == base).all(), exponent


def test_route_select_rejects_more_than_16384_keys(ops, cuda_device):
    with pytest.raises(ValueError, match="16384"):
        ops.route_select(torch.zeros(1, 1, 16385, device=cuda_device), 0.95, 0.625)


@pytest.mark.parametrize("name", ["bootstrap", "prior"])
def test_route_select_matches_reference_at_config3_scale(ops, cuda_device, name):
    """The GPU selection on all 18,000 rows of the route_config3 fixture (40 x
    450 x 450, target .95, cap 282, 29 sink columns, with and without the
    persistence prior) against the reference's own _sampled_route: every row
    with a decision margin above 4 fp32 ulp selects what the reference
    selected (tie order aside), exactly the listed rows differ, and the whole
    route equals the oracle's."""
    from tests.test_oracle_route import CONFIG3_DIFFERENCES, compare_config3, config3_case
    mass, previous, expected, value_sum = config3_case(name)
    route, counts = ops.route_select(
        torch.from_numpy(mass).to(cuda_device), 0.95, 0.625,
        previous=None if previous is None else torch.from_numpy(previous).to(cuda_device),
        persistence=0.5 if previous is not None else 0.0, sink_blocks=29)
    torch.cuda.synchronize()
    got = route.cpu().numpy()
    primed = R.persistence_prior(mass, previous, 0.5) if previous is not None else mass
    oracle, margins = R.top_mass_route(primed, 0.95, 0.625, return_margins=True)
    oracle[..., :29] = True
    assert (got == oracle).all()
    assert (counts.cpu().numpy() == oracle.sum(-1)).all()
    near, tie_order, differing = compare_config3(got, primed, margins, expected, value_sum)
    assert (near, tie_order, differing) == CONFIG3_DIFFERENCES[name]
