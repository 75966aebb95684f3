"""The C-ABI library loads without a GPU, exports every symbol include/qattn.h declares, and its
host-side validation reports errors as status codes (no GPU call is reached on these paths)."""

import ctypes
import os
import re

import pytest

from tests.conftest import ROOT


def _declared():
    src = open(os.path.join(ROOT, "include", "qattn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(qattn_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from telefuser_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libqattn.so not built")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert "qattn_fwd" in names and "qattn_quant_qk_per_block_int8" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_workspace_queries(lib):
    assert lib.qattn_fwd_workspace_size(1, 4680, 12, 128, 1) == 0
    assert lib.qattn_fwd_workspace_size(1, 4680, 12, 128, 4) == 4 * 12 * 4680 * 130 * 4
    assert lib.qattn_seq_mean_workspace_size(1, 32760, 12, 128) == 12 * 128 * 128 * 4
    # the C5 shape (444 query blocks) is split, the C2 shape (3072) is not
    assert lib.qattn_fwd_num_splits(1, 4680, 32760, 12) == 1    # C5: 444 workgroups, splitting costs more
    assert lib.qattn_fwd_num_splits(1, 1024, 32760, 2) > 1      # 16 workgroups: split
    assert lib.qattn_fwd_num_splits(1, 32760, 32760, 12) == 1


def _seq(ptr, sb, sl, sh):
    from telefuser_amd._lib import QattnSeq

    return QattnSeq(ptr, sb, sl, sh)


def test_validation_errors_are_status_codes(lib):
    s = _seq(16, 128 * 128, 128, 128)
    buf = ctypes.c_void_p(16)
    # head ratio
    rc = lib.qattn_fwd(s, buf, s, buf, buf, 128, buf, s, 0, 1, 128, 128, 3, 2, 128, 1.0, 0, 0, None, None, 1, None,
                       0, None)
    assert rc == 6 and b"divisible" in lib.qattn_last_error()
    # head dim
    rc = lib.qattn_fwd(s, buf, s, buf, buf, 128, buf, s, 0, 1, 128, 128, 2, 2, 96, 1.0, 0, 0, None, None, 1, None,
                       0, None)
    assert rc == 5
    # bad dtype in the quantizer
    rc = lib.qattn_quant_per_block_int8(s, 7, 1, 128, 1, 128, None, s, buf, 1.0, 0, 64, 0, None)
    assert rc == 1
    # block size
    rc = lib.qattn_quant_per_block_int8(s, 0, 1, 128, 1, 128, None, s, buf, 1.0, 0, 48, 0, None)
    assert rc == 9
    # misaligned rows
    bad = _seq(16, 128 * 100, 100, 100)
    rc = lib.qattn_quant_per_block_int8(bad, 0, 1, 128, 1, 128, None, s, buf, 1.0, 0, 64, 0, None)
    assert rc == 3
    # missing workspace for a split launch
    rc = lib.qattn_fwd(s, buf, s, buf, buf, 128, buf, s, 0, 1, 128, 128, 2, 2, 128, 1.0, 0, 0, None, None, 2, None,
                       0, None)
    assert rc == 7


def test_fwd_ex_granularity_validation_and_splits(lib):
    s = _seq(16, 128 * 128, 128, 128)
    buf = ctypes.c_void_p(16)

    def call(v_kind, gran, ns=1):
        return lib.qattn_fwd_ex(s, buf, s, buf, buf, v_kind, 128, buf, s, 0, 1, 128, 128, 2, 2, 128, 1.0, gran, 0, 0,
                                None, None, ns, None, 0, None)

    assert call(0, 6) == 9 and b"qk_quant_gran" in lib.qattn_last_error()
    assert call(0, 0) == 9
    # the sm90 tables (codes 4, 5) are per warp / per thread: same split counts as codes 2, 3
    assert lib.qattn_fwd_ex_num_splits(1, 32760, 2000 * 64, 12, 0, 5) == \
        lib.qattn_fwd_ex_num_splits(1, 32760, 2000 * 64, 12, 0, 3)
    assert call(3, 1) == 1
    assert call(1, 3, ns=2) == 7  # a split launch still needs its workspace
    # per-thread K scales take 4x the LDS staging per tile: long keys need more splits
    lk = 2000 * 64
    assert lib.qattn_fwd_ex_num_splits(1, 32760, lk, 12, 0, 3) >= lib.qattn_fwd_ex_num_splits(1, 32760, lk, 12, 0, 1)
    assert lib.qattn_fwd_ex_num_splits(1, 75600, 75600, 40, 0, 3) == 1  # C3 fits one split with FP8 V
    assert lib.qattn_fwd_ex_num_splits(1, 75600, 75600, 40, 1, 3) > 1   # half V leaves less LDS for scales
    assert lib.qattn_fwd_ex_num_splits(1, 4680, 32760, 12, 0, 1) == lib.qattn_fwd_num_splits(1, 4680, 32760, 12)


def test_kernel_selection_rule(lib):
    """qattn_fwd_ex_kernel reports the automatic choice; qattn_set_kernel overrides it per thread."""
    one, multi, pp, res = 1, 2, 3, 4
    assert lib.qattn_fwd_ex_kernel(1, 32760, 32760, 12, 0, 1, 0, 0) == pp      # C2: 1536 ping-pong workgroups
    assert lib.qattn_fwd_ex_kernel(1, 32760, 32760, 12, 0, 3, 0, 0) == pp      # per-thread scales, same rule
    assert lib.qattn_fwd_ex_kernel(1, 75600, 512, 40, 0, 1, 0, 0) == res       # C4: key range fits in LDS
    assert lib.qattn_fwd_ex_kernel(1, 75600, 513, 40, 0, 1, 0, 0) == multi     # 9 tiles: streamed
    assert lib.qattn_fwd_ex_kernel(1, 75600, 512, 40, 0, 1, 1, 0) != res       # causal: resident does not apply
    assert lib.qattn_fwd_ex_kernel(1, 75600, 512, 40, 1, 1, 0, 0) == one       # half P.V
    assert lib.qattn_fwd_ex_kernel(1, 4680, 32760, 12, 0, 1, 0, 0) == pp       # C5: 228 ping-pong workgroups (7/8 of the CUs)
    assert lib.qattn_fwd_ex_kernel(1, 4680, 32760, 11, 0, 1, 0, 0) == pp       # 209 pairs: one round either way
    assert lib.qattn_fwd_ex_kernel(1, 4680, 32760, 8, 0, 1, 0, 0) == pp        # 152 pairs against 296 blocks
    assert lib.qattn_fwd_ex_kernel(1, 2048, 32760, 12, 0, 1, 0, 1) == one      # unsplit, 192 blocks: one per CU
    assert lib.qattn_fwd_ex_kernel(1, 1024, 32760, 2, 0, 1, 0, 0) == pp        # KV split over 8 pairs: ping-pong
    assert lib.qattn_fwd_ex_num_splits(1, 1024, 32760, 2, 0, 1) == 32          # 256 / 8 pairs, at most 32
    assert lib.qattn_fwd_ex_num_splits(1, 4680, 32760, 4, 0, 1) == 3           # 76 pairs -> 228 workgroups
    assert lib.qattn_fwd_ex_kernel(1, 128, 32760, 8, 0, 1, 0, 0) == one        # one block per head: idle pairs
    assert lib.qattn_fwd_ex_kernel(1, 1024, 32760, 2, 1, 1, 0, 0) == one       # half P.V split
    assert lib.qattn_fwd_ex_kernel(1, 1024, 1024, 2, 0, 1, 0, 0) == one        # C1: 16 ping-pong workgroups, too few
    assert lib.qattn_fwd_ex_kernel(1, 32760, 32760, 12, 1, 1, 0, 0) == one     # half P.V
    prev = lib.qattn_set_kernel(pp)
    try:
        assert lib.qattn_fwd_ex_kernel(1, 1024, 1024, 2, 0, 1, 0, 1) == pp
        assert lib.qattn_fwd_ex_kernel(1, 1024, 32760, 2, 0, 1, 0, 0) == pp    # forced: split ping-pong
        assert lib.qattn_fwd_ex_kernel(1, 1024, 32760, 2, 1, 1, 0, 0) == one   # half P.V: no ping-pong form
        lib.qattn_set_kernel(multi)
        assert lib.qattn_fwd_ex_kernel(1, 1024, 1024, 2, 0, 1, 1, 1) == one    # causal: multi-block does not apply
        assert lib.qattn_fwd_ex_kernel(1, 1024, 1024, 2, 0, 1, 0, 1) == multi
        lib.qattn_set_kernel(res)
        assert lib.qattn_fwd_ex_kernel(1, 1024, 1024, 2, 0, 1, 0, 1) == one    # 16 tiles: resident does not apply
        assert lib.qattn_fwd_ex_kernel(1, 1024, 300, 2, 0, 1, 0, 1) == res
        lib.qattn_set_kernel(one)
        assert lib.qattn_fwd_ex_kernel(1, 75600, 512, 40, 0, 1, 0, 0) == one
    finally:
        lib.qattn_set_kernel(prev)
    assert lib.qattn_set_kernel(0) == 0
