"""The CPU oracle against the committed known answers of tests/golden/known_answers.npz (written by
tests/golden/make_golden.py from numpy's correctly rounded float32 arithmetic, hand-derived tree sums and exact
closed forms, without the oracle): quantize_q8_1, rmsnorm_q8 on the tree rows, l2norm_heads on the tree heads,
get_rows_q8_0. Bit-exact. The same file checks the HIP kernels in tests/test_gpu_golden.py."""
import os

import numpy as np
import pytest

from conftest import assert_bits_equal

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "known_answers.npz")
E = 5120
THETA = float(np.float32(1e7) ** np.float32(-2.0 / 64))  # any theta: every angle is 0 in the attn_prep case


@pytest.fixture(scope="module")
def G():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_golden_file_is_current(G):
    """The file holds exactly what the committed generator builds (the generator is deterministic)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(os.path.dirname(GOLD), "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    built = mg.build()
    assert sorted(built) == sorted(G)
    for key, arr in built.items():
        arr = np.asarray(arr)
        assert arr.dtype == G[key].dtype, key
        assert_bits_equal(arr, G[key], key)


def test_golden_cases_are_discriminating(G):
    """The known answers hold the cases they are meant to: ties rounded away from zero, fp16 overflow of d, zero
    blocks, and xs values that a sequential sum would not give."""
    xq, xd = G["q8_xq"].reshape(-1, 32), G["q8_xd"]
    assert np.all(xq[:2] == 0) and np.all(xd[:2] == 0)
    ties = G["q8_x"].reshape(-1, 32)[6:10, 1:]
    assert np.array_equal(np.abs(xq[6:10, 1:]), (np.abs(ties) + 0.5).astype(np.int8))
    assert np.isinf(xd).any()
    xs = G["q8_xs"]
    assert xs[20] == 14.0 and xs[21] == 14.0  # treepins.xs_blocks: sequential sums 7 and 6


def test_quantize_q8_1_golden(oracle, G):
    x = G["q8_x"]
    xq, xd, xs = oracle.quantize_q8_1(x, 256, x.size // 256, with_xs=True)
    assert_bits_equal(xq, G["q8_xq"], "xq")
    assert_bits_equal(xd, G["q8_xd"], "xd")
    assert_bits_equal(xs, G["q8_xs"], "xs")


@pytest.mark.parametrize("i", range(4))
def test_rmsnorm_q8_golden(oracle, G, i):
    h, xq, xd, xs = oracle.rmsnorm_q8(G[f"row{i}_x"], G[f"row{i}_w"], E, 1, float(G[f"row{i}_eps"]), with_xs=True)
    assert_bits_equal(h, G[f"row{i}_h"], f"row {i} h")
    assert_bits_equal(xq, G[f"row{i}_xq"], f"row {i} xq")
    assert_bits_equal(xd, G[f"row{i}_xd"], f"row {i} xd")
    assert_bits_equal(xs, G[f"row{i}_xs"], f"row {i} xs")


@pytest.mark.parametrize("i", range(2))
def test_l2norm_golden(oracle, G, i):
    y = oracle.l2norm_heads(G[f"l2{i}_x"], 128, 1, 1, 128, float(G[f"l2{i}_eps"]))
    assert_bits_equal(y, G[f"l2{i}_y"], f"l2 head {i}")


def test_get_rows_q8_0_golden(oracle, G):
    y = oracle.get_rows("q8_0", G["q80_table"], 34 * (E // 32), G["q80_ids"], E)
    assert_bits_equal(y, G["q80_y"], "q8_0 rows")


def test_attn_prep_golden(oracle, G):
    nb = G["att_kc"].size
    kc, vc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    qn = oracle.attn_prep(G["att_qg"], G["att_k"], G["att_v"], G["att_qw"], G["att_kw"], kc, vc, int(G["att_pos0"]), 4,
                          float(G["att_eps"]), THETA, 24, 4, int(G["att_nctx"]), True, G["att_rope3"])
    assert_bits_equal(qn, G["att_qn"], "qn")
    assert_bits_equal(kc, G["att_kc"], "k cache")
    assert_bits_equal(vc, G["att_vc"], "v cache")
