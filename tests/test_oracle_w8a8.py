"""CPU checks that pin oracle/w8a8.py (closed forms and brute force)."""
import numpy as np

from oracle import w8a8 as o8


def test_acc_kat_all_127():
    K = 14336
    x = np.full((2, K), 127, dtype=np.int8)
    w = np.full((K, 3), 127, dtype=np.int8)
    assert (o8.acc_int32(x, w) == 231225344).all()


def test_acc_alternating_and_min():
    x = np.array([[1, -1, 1, -1], [-128, -128, -128, -128]], dtype=np.int8)
    w = np.array([[127], [127], [-128], [-128]], dtype=np.int8)
    acc = o8.acc_int32(x, w)
    assert acc[0, 0] == 127 - 127 - 128 + 128
    assert acc[1, 0] == -128 * 127 * 2 + 128 * 128 * 2


def test_acc_matches_int64_brute_force():
    rng = np.random.default_rng(0)
    x = rng.integers(-128, 128, (5, 67), dtype=np.int8)
    w = rng.integers(-128, 128, (67, 9), dtype=np.int8)
    want = x.astype(np.int64) @ w.astype(np.int64)
    assert np.array_equal(o8.acc_int32(x, w), want)


def test_epilogue_order_and_rounding():
    """(acc * xs) * ws with fp32 rounding after each product, then fp16 RNE: a case where the
    other association order rounds differently pins the order."""
    rng = np.random.default_rng(1)
    for _ in range(200):
        acc = rng.integers(-2**28, 2**28, (1, 1))
        xs = np.float16(rng.uniform(0.001, 0.011)).reshape(1, 1)
        ws = np.float16(rng.uniform(0.001, 0.011)).reshape(1, 1)
        got = o8.epilogue(acc, xs, ws)[0, 0]
        t = np.float32(np.float32(acc[0, 0]) * np.float32(xs[0, 0]))
        want = np.float16(np.float32(t * np.float32(ws[0, 0])))
        assert got == np.float32(want)
