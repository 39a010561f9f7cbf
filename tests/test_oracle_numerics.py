"""CPU checks pinning oracle/numerics.py against torch's casts (library routines)."""
import numpy as np
import torch

from oracle import numerics as nm


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-30, 100), [0.0, -0.0, 1e38, -3e38]])
    a = a.astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(nm.round_to(a, "bf16"), want)
    # exact ties round to even
    ties = np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8], np.float32)
    assert np.array_equal(nm.round_to(ties, "bf16"), torch.from_numpy(ties).bfloat16().float().numpy())


def test_e4m3_decode_table_matches_torch_exhaustively():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = nm.e4m3fn_decode_table()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x38] == 1.0


def test_e4m3_encoder_matches_torch_on_all_fp16_inputs():
    h = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    f = h.float()
    finite = torch.isfinite(f)
    want = f[finite].to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = nm.e4m3fn_encode_rne(f[finite].numpy())
    wantv = nm.e4m3fn_decode(want)
    gotv = nm.e4m3fn_decode(got)
    both_nan = np.isnan(wantv) & np.isnan(gotv)
    assert np.array_equal(np.where(both_nan, 0, gotv), np.where(both_nan, 0, wantv))


def test_e8m0_kats():
    v = nm.e8m0_decode(np.array([127, 0, 254, 255, 120]))
    assert v[0] == 1.0 and v[1] == 2.0 ** -127 and v[2] == 2.0 ** 127
    assert np.isnan(v[3]) and v[4] == 2.0 ** -7
