"""Pins of the route oracle (CPU): golden vectors written by the reference's own
functions, the reference's known answers, brute-force formulations and
invariants.  Near-tie rows (decision margin <= 4 fp32 ulp) are reported, not
compared, since the reference's torch reductions round in build-specific order.
"""

from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import route as R
from tests.golden.inputs import block_mass_like, clustered_qkv, random_route

GOLDEN = Path(__file__).resolve().parent / "golden"
MARGIN_ULP = 4.0
# dtype code of the sampled_mass fixture -> (input dtype, score rounding).
GOLDEN_DTYPES = {0: (torch.float32, None), 1: (torch.bfloat16, "bf16"),
                 2: (torch.float16, "fp16")}


def _load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def _cases(data):
    return sorted({key.split("__")[0] for key in data.files})


def _compare_routes(actual, expected, margins, mass):
    """Rows must match exactly, except (a) near-tie rows (margin <= 4 ulp) and
    (b) rows that select the same multiset of values, i.e. differ only in which
    of several equal values was taken at the boundary: torch's unstable CPU
    argsort orders equal values arbitrarily, the oracle by index ascending.
    Returns (near-tie rows, tie-order rows, mismatched rows)."""
    safe = margins.reshape(-1) > MARGIN_ULP
    a = actual.reshape(-1, actual.shape[-1])
    e = expected.reshape(-1, expected.shape[-1])
    values = np.asarray(mass, dtype=np.float32).reshape(a.shape)
    mismatched = np.nonzero((a != e).any(-1))[0]
    tie_order = 0
    for row in mismatched:
        same_values = np.array_equal(np.sort(values[row][a[row]]), np.sort(values[row][e[row]]))
        tie_order += int(same_values)
        assert same_values or not safe[row], f"row {row} differs with a safe margin"
    return int((~safe).sum()), tie_order, int(mismatched.size)


def test_known_answer_row_cap():
    """tests/test_flex_backend.py:56-59."""
    mass = np.array([[[0.50, 0.30, 0.15, 0.05]]], np.float32)
    assert R.top_mass_route(mass, 0.90, 0.50).tolist() == [[[True, True, False, False]]]


@pytest.mark.parametrize("case", _cases(_load("top_mass_route")))
def test_top_mass_matches_reference_golden(case):
    data = _load("top_mass_route")
    mass = data[f"{case}__mass"]
    target, keep = data[f"{case}__params"]
    route, margins = R.top_mass_route(mass, target, keep, return_margins=True)
    near, tie_order, mismatched = _compare_routes(route, data[f"{case}__route"], margins, mass)
    assert mismatched <= near + tie_order
    # Selected-block counts are order independent and must always agree.
    assert (route.sum(-1) == data[f"{case}__route"].sum(-1)).all() or near > 0


def test_tie_order_is_index_ascending_like_a_stable_sort():
    """Ties are broken by key index ascending: the order of a stable
    descending sort (torch.argsort(stable=True), CUDA's radix sort)."""
    data = _load("top_mass_route")
    mass = data["ties__mass"]
    target, keep = data["ties__params"]
    route = R.top_mass_route(mass, target, keep)
    order = torch.argsort(torch.from_numpy(mass), dim=-1, descending=True, stable=True)
    counts = torch.from_numpy(route.sum(-1))
    ranks = torch.empty_like(order).scatter_(-1, order, torch.arange(mass.shape[-1]).expand_as(order))
    assert (ranks < counts.unsqueeze(-1)).numpy().tolist() == route.tolist()


def _brute_force_count(row, target, cap):
    """Fewest top blocks whose exact (rational) mass reaches target * total."""
    order = sorted(range(len(row)), key=lambda i: (-row[i], i))
    values = [Fraction(float(row[i])) for i in order]
    threshold = Fraction(float(np.float32(target))) * sum(values)
    running = Fraction(0)
    for count, value in enumerate(values, start=1):
        running += value
        if running >= threshold:
            return min(count, cap), order
    return min(len(values), cap), order


def test_top_mass_matches_brute_force_on_safe_rows():
    rng = np.random.default_rng(5)
    mass = rng.dirichlet(np.full(40, 0.4), size=60).astype(np.float32)
    mass[:5] = np.round(mass[:5] * 16) / 16  # exact ties
    route, margins = R.top_mass_route(mass, 0.9, 0.6, return_margins=True)
    cap = R.route_cap(40, 0.6)
    for row in range(mass.shape[0]):
        if margins[row] <= MARGIN_ULP:
            continue
        count, order = _brute_force_count(mass[row], 0.9, cap)
        expected = np.zeros(40, dtype=bool)
        expected[order[:count]] = True
        assert (route[row] == expected).all(), row


def test_planted_mistakes_are_caught_by_golden():
    """Mutations of the oracle (count without +1, ties by index descending)
    must disagree with the reference's golden routes."""
    data = _load("top_mass_route")

    def off_by_one(mass, target, keep):
        rows = mass.reshape(-1, mass.shape[-1]).astype(np.float64)
        order = np.argsort(-rows, axis=-1, kind="stable")
        prefix = np.cumsum(np.take_along_axis(rows, order, -1), -1)
        counts = np.minimum((prefix < rows.sum(-1, keepdims=True) * target).sum(-1),
                            R.route_cap(rows.shape[-1], keep))
        ranks = np.argsort(order, -1)
        return (ranks < counts[:, None]).reshape(mass.shape)

    def ties_descending(mass, target, keep):
        flipped = mass[..., ::-1]
        return R.top_mass_route(flipped, target, keep)[..., ::-1]

    for mutant in (off_by_one, ties_descending):
        differs = False
        for case in ("dirichlet", "ties"):
            target, keep = data[f"{case}__params"]
            got = mutant(data[f"{case}__mass"], target, keep)
            differs |= bool((got != data[f"{case}__route"]).any())
        assert differs, mutant.__name__


def test_persistence_prior_and_sampled_route_golden():
    """FlexReuseBackend._sampled_route with a previous route (flex.py:535-548)."""
    data = _load("sampled_route")
    mass = data["mass"]
    primed = R.persistence_prior(mass, data["previous"], 0.5)
    route, margins = R.top_mass_route(primed, 0.95, 0.625, return_margins=True)
    near, tie_order, mismatched = _compare_routes(route, data["route"], margins, primed)
    assert mismatched <= near + tie_order
    # The prior only ever adds mass to previously routed blocks.
    assert (primed >= mass).all()
    assert (primed[~data["previous"]] == mass[~data["previous"]]).all()


def test_prior_is_exact_closed_form_on_dyadic_rows():
    mass = np.array([[0.5, 0.25, 0.125, 0.125]], np.float32)
    previous = np.array([[False, True, False, True]])
    # mean = 0.25, rho * mean = 0.125.
    expected = np.array([[0.5, 0.375, 0.125, 0.25]], np.float32)
    assert (R.persistence_prior(mass, previous, 0.5) == expected).all()


@pytest.mark.parametrize("case", _cases(_load("sampled_mass")))
def test_sampled_mass_matches_reference_golden(case):
    data = _load("sampled_mass")
    tokens, heads, dim, block, samples, code, seed = (int(x) for x in data[f"{case}__params"])
    dtype, score_dtype = GOLDEN_DTYPES[code]
    q, k, _ = clustered_qkv(tokens, heads, dim, group=block, seed=seed, dtype=dtype)
    np.testing.assert_allclose(
        [q.double().sum().item(), k.double().sum().item()], data[f"{case}__checksum"])
    mass = R.sampled_block_mass(q.float().numpy(), k.float().numpy(), block, samples,
                                score_dtype=score_dtype, bf16_scores=False)
    expected = data[f"{case}__mass"]
    tolerance = 2e-3 if score_dtype else 2e-6
    np.testing.assert_allclose(mass, expected, atol=tolerance, rtol=tolerance)
    np.testing.assert_allclose(mass.sum(-1), 1.0, atol=1e-9)


def test_sampled_mass_query_block_subset_equals_full_rows():
    """The row-restricted form (used at full config-3 scale) returns exactly
    the selected rows of the full computation, in the order asked for, and
    still matches the reference golden on them."""
    data = _load("sampled_mass")
    tokens, heads, dim, block, samples, _, seed = (
        int(x) for x in data["bf16_partial_s16__params"])
    q, k, _ = clustered_qkv(tokens, heads, dim, group=block, seed=seed, dtype=torch.bfloat16)
    qn, kn = q.float().numpy(), k.float().numpy()
    full = R.sampled_block_mass(qn, kn, block, samples)
    blocks = full.shape[1]
    subset = [blocks - 1, 0, blocks // 2]
    rows = R.sampled_block_mass(qn, kn, block, samples, query_blocks=subset)
    assert rows.shape == (heads, len(subset), blocks)
    np.testing.assert_array_equal(rows, full[:, subset])
    np.testing.assert_allclose(rows, data["bf16_partial_s16__mass"][:, subset],
                               atol=2e-3, rtol=2e-3)


def test_full_sampling_matches_exact_block_mass():
    """tests/test_flex_backend.py:43-53: samples == block gives exact / block."""
    rng = np.random.default_rng(4)
    tokens, heads, dim, block = 12, 2, 8, 4
    q = rng.standard_normal((1, tokens, heads, dim)).astype(np.float32)
    k = rng.standard_normal((1, tokens, heads, dim)).astype(np.float32)
    scores = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), k.astype(np.float64))
    scores *= dim ** -0.5
    probabilities = np.exp(scores - scores.max(-1, keepdims=True))
    probabilities /= probabilities.sum(-1, keepdims=True)
    exact = probabilities[0].reshape(heads, 3, block, 3, block).sum((2, 4))
    sampled = R.sampled_block_mass(q, k, block, samples=block, bf16_scores=False)
    np.testing.assert_allclose(sampled, exact / block, atol=1e-6, rtol=1e-6)


def test_sample_indices_known_answers():
    indices, sizes = R.sample_indices(300, 128, 16)
    assert indices[0].tolist() == list(range(4, 128, 8))
    assert sizes.tolist() == [128, 128, 44]
    # Partial block of 44 tokens: floor((2s+1)*44/32).
    assert indices[2].tolist() == [256 + (2 * s + 1) * 44 // 32 for s in range(16)]


def test_pack_rows_known_answer_and_stable_partition():
    """tests/test_flex_backend.py:16-40."""
    route = np.array([[[True, False, True], [False, True, False]],
                      [[False, True, True], [True, False, True]]])
    counts, indices = R.pack_rows(route)
    assert counts.tolist() == [[2, 1], [2, 2]]
    rng = np.random.default_rng(19)
    route = rng.random((5, 37, 450)) < 0.61
    counts, indices = R.pack_rows(route)
    expected = torch.argsort(torch.from_numpy(route).to(torch.int8), dim=-1,
                             descending=True, stable=True).numpy()
    assert (indices == expected).all()
    assert (counts == route.sum(-1)).all()


def test_csr_round_trip():
    rng = np.random.default_rng(2)
    route = rng.random((3, 9, 9)) < 0.5
    row_ptr, col_idx, counts = R.to_csr(route)
    rebuilt = np.zeros_like(route).reshape(-1, 9)
    for row in range(rebuilt.shape[0]):
        rebuilt[row, col_idx[row_ptr[row]:row_ptr[row + 1]]] = True
    assert (rebuilt.reshape(route.shape) == route).all()
    assert (np.diff(row_ptr) == counts.reshape(-1)).all()


def test_first_frame_sink_known_answer():
    """tests/test_flex_route_update.py:106-112: grid (2,8,16) -> column 0 only."""
    route = R.first_frame_sink(np.zeros((2, 4, 4), dtype=bool), (2, 8, 16), 128)
    assert route[..., 0].all() and not route[..., 1:].any()
    assert R.first_frame_sink(np.zeros((1, 1, 450), bool), (16, 45, 80), 128).sum() == 29


def test_dispatch_keep_threshold():
    """tests/test_flex_route_update.py:41-73: an all-ones route, threshold .75."""
    assert R.dense_dispatch(np.ones((1, 1, 1), bool), 0.75)
    assert not R.dense_dispatch(np.eye(4, dtype=bool)[None], 0.75)
    assert R.route_keep(np.eye(4, dtype=bool)[None]) == 0.25


def route_fingerprint(route, values):
    """Per-row (count, sum of selected indices, sum of their squares) of a
    boolean route, and the float64 sum of the selected ``values``."""
    route = np.asarray(route, dtype=bool)
    index = np.arange(route.shape[-1], dtype=np.int64)
    return ((route.sum(-1), (route * index).sum(-1), (route * index * index).sum(-1)),
            (np.asarray(values, dtype=np.float64) * route).sum(-1))


def config3_case(name):
    """Mass, previous route (or None) and the reference's fingerprints and
    selected-value sums of the route_config3 fixture (make_golden.py)."""
    data = _load("route_config3")
    heads, blocks, seed, sharpness, previous_seed = data["params"]
    mass = block_mass_like(int(heads), int(blocks), int(seed), sharpness=float(sharpness)).numpy()
    previous = random_route(int(heads), int(blocks), int(previous_seed)).numpy()
    expected = tuple(data[f"{name}__{key}"] for key in ("count", "index_sum", "square_sum"))
    return mass, (previous if name == "prior" else None), expected, data[f"{name}__value_sum"]


def compare_config3(route, primed, margins, expected, value_sum):
    """Rows whose decision margin exceeds 4 fp32 ulp must select what the
    reference selected: the same blocks, or, where torch's unstable argsort
    took another of several equal boundary values, the same count and the
    same sum of selected values.  Returns (near-tie rows, tie-order rows,
    differing rows)."""
    indices, values = route_fingerprint(route, primed)
    same = np.all([g == e for g, e in zip(indices, expected)], axis=0)
    tie_order = ~same & (indices[0] == expected[0]) & (values == value_sum)
    safe = margins > MARGIN_ULP
    assert (same | tie_order)[safe].all(), np.argwhere(safe & ~same & ~tie_order)[:5]
    return int((~safe).sum()), int(tie_order.sum()), int((~same).sum())


# Rows of the route_config3 fixture (18,000 rows each) that are near ties
# (decision margin <= 4 fp32 ulp), that select tied values in another order
# (same count, same selected sum), and that differ from the reference's own
# route at all.  Bootstrap: the one differing row is (head 18, query block
# 376), 228 blocks here against 227, at a 1-ulp margin, where the reference's
# count depends on torch's fp32 summation order.  Prior: the one differing row
# is (11, 199), the same 294 blocks and selected sum in another tie order.
CONFIG3_DIFFERENCES = {"bootstrap": (16, 0, 1), "prior": (10, 1, 1)}


@pytest.mark.parametrize("name", ["bootstrap", "prior"])
def test_oracle_matches_reference_route_at_config3_scale(name):
    """All 18,000 rows of a 40 x 450 x 450 selection (target .95, cap 282,
    29 sink columns) against the reference's _sampled_route on the same mass
    (and, for "prior", the same previous route and persistence 0.5)."""
    mass, previous, expected, value_sum = config3_case(name)
    primed = R.persistence_prior(mass, previous, 0.5) if previous is not None else mass
    route, margins = R.top_mass_route(primed, 0.95, 0.625, return_margins=True)
    route[..., :29] = True
    near, tie_order, differing = compare_config3(route, primed, margins, expected, value_sum)
    assert (near, tie_order, differing) == CONFIG3_DIFFERENCES[name]


@pytest.mark.parametrize("prior", [False, True])
def test_route_is_invariant_to_power_of_two_scaling(prior):
    """Top-mass selection depends only on the ratios of a row's values, so a
    power-of-two scale of the mass (exact in fp32) must not change the route,
    including scales whose row sums are far above the 2^11 a fixed 2^52 fixed
    point holds and far below fp32's normal range of sums."""
    rng = np.random.default_rng(7)
    mass = rng.dirichlet(np.full(450, 0.4), size=(4, 32)).astype(np.float32)
    previous = rng.random(mass.shape) < 0.6 if prior else None
    base = R.sampled_route(None, None, 128, 16, 0.95, 0.625, previous=previous, rho=0.5,
                           mass=mass)
    for exponent in (-90, -20, 12, 40):
        scaled = np.ldexp(mass, exponent).astype(np.float32)
        got = R.sampled_route(None, None, 128, 16, 0.95, 0.625, previous=previous, rho=0.5,
                              mass=scaled)
        assert (got == base).all(), exponent


def test_row_shift_bounds_every_sum():
    """K * max * 2^s < 2^10 <= 2 K * max * 2^s: sums of a row's fixed-point
    images stay below 2^62, and s is the largest such exponent."""
    rng = np.random.default_rng(8)
    for keys in (1, 450, 2048, 16384):
        mass = (rng.random((6, keys)) * np.float32(10.0) ** rng.integers(-30, 30, (6, 1))
                ).astype(np.float32)
        shift = R.row_shift(mass)
        bound = keys * mass.max(-1).astype(np.float64) * np.ldexp(1.0, shift)
        assert (bound < 2 ** 10).all() and (2 * bound >= 2 ** 10).all()
        fixed = R._fixed(mass, shift[:, None])
        assert (fixed.sum(-1) < 2 ** 62).all()
