"""C-ABI checks that need no GPU: every function declared in include/dsa.h is
exported by libdsa.so and bound in the ctypes table, and argument validation
(which runs on the host before any HIP call) reports the documented errors."""

import ctypes
import re
from pathlib import Path

import pytest

from dit_sparse_atten_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "dsa.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIBRARY_PATH.exists():
        pytest.skip("libdsa.so not built")
    return _lib.load()


def test_header_symbols_are_exported_and_bound(lib):
    declared = _declared()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes binding"
    assert set(_lib.SIGNATURES) == set(declared)


def test_version_and_workspace_size(lib):
    assert lib.dsa_version() == 1
    # The workspace holds the work-queue counter (256 bytes), the launch order
    # of a routed call (4 bytes per (batch, head, query block) work item,
    # rounded up to 256), the aligned-walk table (8 XCDs x 64 entries of 8
    # bytes) and 64 key-norm maxima per (batch, head) (fp32, rounded up to
    # 256; none above 4,096 pairs), then the split partials of the last round,
    # 1,024 workgroups of 128 x (128 + 2) fp32, when the key range can be
    # split (at least 16 key blocks, 2 parts of 8).  V is read in place.
    def order(items, pairs):
        norms = (pairs * 64 * 4 + 255) // 256 * 256 if pairs <= 4096 else 0
        return 256 + (items * 4 + 255) // 256 * 256 + 8 * 64 * 8 + norms

    split = 1024 * (128 * 128 + 256) * 4
    assert lib.dsa_bsa_workspace_bytes(2, 12, 32760, 128) == order(2 * 12 * 256, 24) + split
    assert lib.dsa_bsa_workspace_bytes(1, 40, 57600, 128) == order(40 * 450, 40) + split
    assert lib.dsa_bsa_workspace_bytes_block(1, 1, 16 * 72, 128, 72) == order(16, 1) + split
    # Key ranges too short to split need the front only: 512 text tokens (4
    # blocks), 10 blocks of 72 tokens, one 1-token block.
    assert lib.dsa_bsa_workspace_bytes(1, 12, 512, 128) == order(12 * 4, 12)
    assert lib.dsa_bsa_workspace_bytes_block(1, 1, 720, 128, 72) == order(10, 1)
    assert lib.dsa_bsa_workspace_bytes_block(1, 1, 1, 128, 1) == order(1, 1)
    # 8,192 (batch, head) pairs: ordered, without norms.
    assert lib.dsa_bsa_workspace_bytes(64, 128, 256, 128) == order(64 * 128 * 2, 8192)
    # More than 262,144 work items run in launch order: no front bytes.
    assert lib.dsa_bsa_workspace_bytes_block(1, 64, 8192 * 8, 128, 8) == split
    assert lib.dsa_bsa_workspace_bytes(0, 12, 10, 128) == 0


def test_invalid_arguments_are_reported_before_any_launch(lib):
    strides = _lib.int64_array([8] * 12)
    status = lib.dsa_bsa_fwd(None, None, None, None, 0, strides, 1, 128, 128, 1, 128, 128,
                             None, None, 1, 0.1, 0, 0, None, None, 0, None)
    assert status == _lib.DSA_EINVAL
    assert "null" in _lib.last_error()
    with pytest.raises(ValueError, match="null"):
        _lib.check(status, "dsa_bsa_fwd")
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 264, 128,
                             None, None, 1, 0.1, 0, 0, None, fake, 1 << 20, None)
    assert status == _lib.DSA_EUNSUPPORTED and "head_dim" in _lib.last_error()
    misaligned = ctypes.c_void_p(24)
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 128, 128,
                             None, None, 1, 0.1, 0, 0, None, misaligned, 1 << 20, None)
    assert status == _lib.DSA_EINVAL and "workspace" in _lib.last_error()
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 128, 128,
                             None, None, 1, 0.1, 0, 0, None, None, 1 << 20, None)
    assert status == _lib.DSA_EINVAL and "workspace" in _lib.last_error()
    status = lib.dsa_route_select(fake, None, 4, 16385, 0.5, 0.95, 1, 0, fake, fake, None)
    assert status == _lib.DSA_EUNSUPPORTED and "16384" in _lib.last_error()
    status = lib.dsa_sampled_mass(fake, fake, 0, _lib.int64_array([8] * 4), 1024, 2, 128, 128,
                                  129, 0.1, fake, None)
    assert status == _lib.DSA_EINVAL and "route_samples" in _lib.last_error()
    status = lib.dsa_sampled_mass(fake, fake, 2, _lib.int64_array([8] * 4), 1024, 2, 128, 128,
                                  16, 0.1, fake, None)
    assert status == _lib.DSA_EUNSUPPORTED and "dtype" in _lib.last_error()
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 7, strides, 1, 128, 128, 1, 128, 128,
                             None, None, 1, 0.1, 0, 0, None, None, 0, None)
    assert status == _lib.DSA_EUNSUPPORTED and "dtype" in _lib.last_error()
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 128, 128,
                             fake, fake, 1, 0.1, 1, 0, None, None, 0, None)
    assert status == _lib.DSA_EUNSUPPORTED and "causal" in _lib.last_error()
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 128, 128,
                             None, None, 1, 0.1, 2, 0, None, None, 0, None)
    assert status == _lib.DSA_EINVAL and "causal" in _lib.last_error()
    status = lib.dsa_bsa_fwd(fake, fake, fake, fake, 0, strides, 1, 128, 128, 1, 128, 128,
                             fake, fake, 1, 0.1, 0, 2, None, None, 0, None)
    assert status == _lib.DSA_EINVAL and "deterministic" in _lib.last_error()
    status = lib.dsa_permute_rows(4, None, None, None, None, None, 1, 1, 1, 16, None)
    assert status == _lib.DSA_EINVAL


def test_exact_and_routing_entry_points_validate_first(lib):
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    strides = _lib.int64_array([8] * 4)
    status = lib.dsa_block_mass(fake, fake, 0, strides, 256, 2, 60, 128, fake, 256, 0.1, fake, None)
    assert status == _lib.DSA_EUNSUPPORTED and "head_dim" in _lib.last_error()
    status = lib.dsa_block_mass(fake, fake, 0, strides, 256, 2, 128, 128, fake, 100, 0.1, fake,
                                None)
    assert status == _lib.DSA_EINVAL and "lse" in _lib.last_error()
    status = lib.dsa_block_mass(fake, fake, 0, strides, 256, 2, 128, 128, fake, 256, -1.0, fake,
                                None)
    assert status == _lib.DSA_EINVAL and "scale" in _lib.last_error()
    aligned = ctypes.c_void_p(4096)
    status = lib.dsa_frontier_mask(fake, 2, 16385, fake, fake, None, None)
    assert status == _lib.DSA_EUNSUPPORTED and "16384" in _lib.last_error()
    status = lib.dsa_directional_update(fake, fake, None, fake, 1, 16385, 8, 0.5, 0.0, 0.0, 1.0,
                                        0, 7, 0, fake, fake, aligned, None, None, None, None)
    assert status == _lib.DSA_EUNSUPPORTED and "16384" in _lib.last_error()
    status = lib.dsa_tile_stats(fake, fake, 0, strides, 16385, 1, 128, 1, 1, fake, 16385, None,
                                None, 0.1, fake, None, None, None, None, None, None)
    assert status == _lib.DSA_EUNSUPPORTED and "16384" in _lib.last_error()
    status = lib.dsa_frontier_mask(fake, 2, 16, None, fake, None, None)
    assert status == _lib.DSA_EINVAL and "neighbors" in _lib.last_error()
    aligned = ctypes.c_void_p(4096)
    status = lib.dsa_directional_update(fake, fake, None, fake, 2, 16, 0, 0.5, 0.0, 0.0, 1.0,
                                        0, 7, 0, fake, fake, aligned, None, None, None, None)
    assert status == _lib.DSA_EINVAL and "cap" in _lib.last_error()
    status = lib.dsa_directional_update(fake, fake, None, fake, 2, 16, 8, 0.5, 0.0, 0.0, 0.0,
                                        0, 7, 0, fake, fake, aligned, None, None, None, None)
    assert status == _lib.DSA_EINVAL and "budget_scale" in _lib.last_error()
    status = lib.dsa_directional_update(fake, fake, None, fake, 2, 16, 8, 0.5, 0.0, 0.0, 1.0,
                                        0, 7, 0, fake, fake, ctypes.c_void_p(4097), None, None,
                                        None, None)
    assert status == _lib.DSA_EINVAL and "aligned" in _lib.last_error()


def test_tile_stats_validates_first(lib):
    fake = ctypes.c_void_p(16)
    strides = _lib.int64_array([8] * 4)
    status = lib.dsa_tile_stats(fake, fake, 0, strides, 1024, 2, 128, 12, 12, fake, 1024, None,
                                None, 0.1, fake, None, None, None, None, None, None)
    assert status == _lib.DSA_EUNSUPPORTED and "128" in _lib.last_error()
    status = lib.dsa_tile_stats(fake, fake, 0, strides, 1000, 2, 128, 8, 8, fake, 1000, None,
                                None, 0.1, fake, None, None, None, None, None, None)
    assert status == _lib.DSA_EINVAL and "whole" in _lib.last_error()
    status = lib.dsa_tile_stats(fake, fake, 0, strides, 1024, 2, 128, 8, 8, fake, 1024, fake,
                                None, 0.1, fake, None, None, None, None, None, None)
    assert status == _lib.DSA_EINVAL
