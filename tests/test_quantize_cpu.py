"""CPU checks of the activation quantizer (the step before the operator): the oracle
restatement of kernel.cu:998-1062 is pinned against things it shares no code with,
and the C-ABI entry point's argument checks run without a GPU.

* the e4m3 encoder against torch's float8_e4m3fn cast on every code, every midpoint
  between neighbouring codes (ties), values one ulp either side of each midpoint,
  subnormals, signed zeros and random values; a planted ties-away-from-zero encoder
  fails the midpoint check;
* closed forms of the quantizer: constant blocks give +-448 with scale |c|/448, an
  all-zero block gives scale 1 and zero codes, a block of exactly representable
  values with absmax 448 * 2^k comes back code for code with scale 2^k, NaN is
  ignored by the absmax and becomes -448; a planted one-absmax-per-row quantizer
  fails on a row of blocks of different magnitudes;
* x * (1/scale) as the reference writes it, not x / scale: a searched input where
  the two give different codes pins which one the oracle follows;
* the round trip |e4m3(q) * scale - x| <= 2^-4 |x| + 2^-10 scale on random rows.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import oracle, pkg


def _torch_e4m3(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _encoder_cases() -> np.ndarray:
    o = oracle()
    tab = o.e4m3_table()[:127].astype(np.float32)
    mid = ((tab[:-1].astype(np.float64) + tab[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))])
    rng = np.random.default_rng(5)
    rnd = np.concatenate([rng.standard_normal(20000) * 40, rng.standard_normal(5000) * 2.0 ** -8,
                          rng.uniform(-448, 448, 5000)]).astype(np.float32).clip(-448, 448)
    v = np.concatenate([tab, mid, near, rnd, np.array([0.0, 2.0 ** -10, 2.0 ** -11, 448.0], np.float32)])
    return np.concatenate([v, -v]).astype(np.float32)


def test_e4m3_encoder_matches_torch_cast():
    v = _encoder_cases()
    assert np.array_equal(oracle().e4m3_encode_rne(v), _torch_e4m3(v))
    assert oracle().e4m3_encode_rne(np.array([-0.0], np.float32))[0] == 0x80


def test_planted_ties_away_encoder_fails_the_midpoints():
    o = oracle()
    tab = o.e4m3_table()[:127].astype(np.float64)
    mid = ((tab[:-1] + tab[1:]) / 2).astype(np.float32)
    assert not np.array_equal(o.e4m3_encode_rne(mid, _ties="away"), _torch_e4m3(mid))


def test_quantizer_closed_forms():
    o = oracle()
    x = np.zeros((3, 512), np.float32)
    x[0, :128] = 3.0                     # constant block
    x[0, 128:256] = -0.75                # constant negative block
    # block 2: all zero
    tab = o.e4m3_table()[:127].astype(np.float32)
    codes = np.arange(128) % 127
    x[0, 384:512] = tab[codes] * 4.0     # exact values, absmax 448 * 4
    x[0, 384] = 448.0 * 4.0
    q, s = o.quantize_fp8_blockwise(x)
    assert s.shape == (4, 3)
    assert np.all(q[0, :128] == 0x7E) and s[0, 0] == np.float32(3.0) / np.float32(448.0)
    assert np.all(q[0, 128:256] == 0xFE) and s[1, 0] == np.float32(0.75) / np.float32(448.0)
    assert np.all(q[0, 256:384] == 0) and s[2, 0] == 1.0
    expect = codes.astype(np.uint8).copy()
    expect[0] = 0x7E
    assert s[3, 0] == 4.0 and np.array_equal(q[0, 384:512], expect)
    # rows of zeros: scale 1 everywhere
    assert np.all(s[:, 1] == 1.0) and np.all(q[1] == 0)


def test_quantizer_nan_and_signed_zero():
    o = oracle()
    x = np.full((1, 128), 2.0, np.float32)
    x[0, 5] = np.nan
    x[0, 6] = -0.0
    x[0, 7] = 896.0
    q, s = o.quantize_fp8_blockwise(x)
    assert s[0, 0] == np.float32(896.0) / np.float32(448.0)     # NaN ignored by the absmax
    assert q[0, 5] == 0xFE                                       # NaN -> fmaxf(.., -448) -> -448
    assert q[0, 6] == 0x80 and q[0, 7] == 0x7E


def test_planted_row_absmax_fails():
    o = oracle()
    x = np.ones((1, 256), np.float32)
    x[0, 128:] = 1000.0
    good, _ = o.quantize_fp8_blockwise(x)
    bad, _ = o.quantize_fp8_blockwise(x, _block_amax=False)
    assert np.all(good == 0x7E)
    assert not np.array_equal(good, bad)


def test_reciprocal_multiply_not_division():
    """Find (x, absmax) where e4m3(x * (1/s)) != e4m3(x / s) and check the oracle takes
    the reciprocal form, as kernel.cu:1038 and 1048 do.  The two products differ by at
    most an fp32 ulp, so the search puts x within a few ulps of s times an e4m3
    rounding midpoint."""
    o = oracle()
    tab = o.e4m3_table()[:127].astype(np.float64)
    mids = ((tab[:-1] + tab[1:]) / 2)[40:]          # midpoints between 1/16 and 448
    rng = np.random.default_rng(11)
    found = None
    for _ in range(4000):
        amax = np.float32(rng.uniform(0.5, 4.0))
        s = np.float32(amax / np.float32(448.0))
        inv = np.float32(np.float32(1.0) / s)
        m = mids[rng.integers(len(mids))]
        base = np.float32(m * float(s))
        xs = np.array([base], np.float32)
        for _ in range(4):
            xs = np.concatenate([xs, np.nextafter(xs, np.float32(np.inf)), np.nextafter(xs, np.float32(-np.inf))])
        xs = np.unique(xs[np.abs(xs) <= amax])
        a = _torch_e4m3(np.clip((xs * inv).astype(np.float32), -448, 448))
        b = _torch_e4m3(np.clip((xs / s).astype(np.float32), -448, 448))
        diff = np.nonzero(a != b)[0]
        if diff.size:
            found = (amax, xs[diff[0]], a[diff[0]], b[diff[0]])
            break
    assert found is not None, "no distinguishing input found"
    amax, xv, code_recip, code_div = found
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = amax
    x[0, 1] = xv
    q, _ = o.quantize_fp8_blockwise(x)
    assert q[0, 1] == code_recip and q[0, 1] != code_div


def test_round_trip_bound():
    o = oracle()
    x = (torch.randn(16, 1024, generator=torch.Generator().manual_seed(2)) *
         torch.logspace(-6, 3, 16).unsqueeze(1)).to(torch.bfloat16)
    q, s = o.quantize_fp8_blockwise(x)
    deq = o.e4m3_table()[q.astype(np.int64)] * np.repeat(s.T, 128, axis=1)
    xf = x.float().numpy()
    bound = 2.0 ** -4 * np.abs(xf) + 2.0 ** -10 * np.repeat(s.T, 128, axis=1)
    assert np.all(np.abs(deq - xf) <= bound * (1 + 1e-6))


@pytest.fixture(scope="module")
def lib():
    return pkg("kernel")._build_extension()


def test_quantize_entry_rejects_bad_arguments_without_a_gpu(lib):
    f = lib.moe_mi355_quantize_fp8_blockwise
    assert f(None, 1, 4, 100, None, None, None) == -2          # cols not a multiple of 128
    assert f(None, 1, 4, 0, None, None, None) == -2
    assert f(None, 1, 4, 65536, None, None, None) == -2        # above the column limit
    assert f(None, 7, 4, 128, None, None, None) == -2          # unknown dtype
    assert f(None, 1, -1, 128, None, None, None) == -2
    assert f(None, 1, 0, 128, None, None, None) == 0           # nothing to do
    assert f(None, 1, 4, 128, None, None, None) == -1          # NULL tensors
    fake = 1 << 20
    assert f(ctypes.c_void_p(fake + 8), 1, 4, 128, ctypes.c_void_p(fake), ctypes.c_void_p(fake), None) == -4


def test_python_wrapper_validates():
    k = pkg("kernel")
    with pytest.raises(ValueError):
        k.quantize_fp8_blockwise(torch.zeros(4, 100, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        k.quantize_fp8_blockwise(torch.zeros(4, 128, dtype=torch.float16))
    with pytest.raises(ValueError):
        k.quantize_fp8_blockwise(torch.zeros(4, 128, dtype=torch.bfloat16))   # host tensor
