"""Quantize-on-append at the rounding boundaries, byte for byte against the CPU checker.

The append's int8 and fp8 quantizers compute y = x * (1/s) and keep the divide x / s only where y lies within
8 ulps of a rounding boundary of the target format (int8: the half-integers; e4m3: the midpoints between
neighbouring codes, and the whole subnormal range); fp8 codes of the other values (infinite ones included: they
clamp to 448, as the conversion saturates) come from the hardware conversion.
These cases put fp32 source values on, and a few ulps to either side of, every such boundary and every e4m3
code, plus values at and beyond the saturation point, subnormal-range values, signed zeros, infinities and NaN,
so that both paths and their seam are exercised.  Pages and int8 scales must equal the checker's bytes.
"""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

D = 128


def _neighbours(v: np.ndarray, ulps=(0, 1, 2, 3, 5, 7, 8, 9, 10, 16, 17, 63, 64, 65, 66, 70, 200)) -> np.ndarray:
    """v and the fp32 values `ulps` steps above and below it."""
    out = [v]
    for k in ulps[1:]:
        up, dn = v.copy(), v.copy()
        for _ in range(k):
            up = np.nextafter(up, np.float32(np.inf)).astype(np.float32)
            dn = np.nextafter(dn, np.float32(-np.inf)).astype(np.float32)
        out += [up, dn]
    return np.concatenate(out).astype(np.float32)


def _rows(vals: np.ndarray, rng) -> np.ndarray:
    """Pad to whole rows of D values (shuffled so each row mixes cases)."""
    vals = rng.permutation(vals)
    n = -(-vals.size // D) * D
    out = np.zeros(n, np.float32)
    out[:vals.size] = vals
    return out.reshape(-1, D)


def _run(ff, gpu, rows_k: np.ndarray, rows_v: np.ndarray, cache: str, head_scale=None):
    import torch

    T = rows_k.shape[0]
    k_src = rows_k.reshape(1, T, 1, D)
    v_src = rows_v.reshape(1, T, 1, D)
    N = -(-T // 16) + 1
    table = np.arange(N, dtype=np.int32)[::-1].copy().reshape(1, N)  # pages in reverse order
    dt = O.DTYPE_I8 if cache == "i8" else O.DTYPE_FP8
    store = np.int8 if cache == "i8" else np.uint8
    hk = np.full((N, 16, 1, D), 0x5A, np.uint8).view(store)
    hv = hk.copy()
    if cache == "i8":
        hks = np.full((N, 16, 1), -1.0, np.float32)
        hvs = hks.copy()
    else:
        hks = np.array([head_scale[0]], np.float32)
        hvs = np.array([head_scale[1]], np.float32)
    dk, dv = torch.from_numpy(hk.copy()).to(gpu), torch.from_numpy(hv.copy()).to(gpu)
    dks, dvs = torch.from_numpy(hks.copy()).to(gpu), torch.from_numpy(hvs.copy()).to(gpu)
    print(f"case quantize edges cache={cache} tokens={T}", flush=True)
    ff.append_kv_cache(torch.from_numpy(k_src).to(gpu), torch.from_numpy(v_src).to(gpu), dk, dv,
                       torch.from_numpy(table).to(gpu), None, dks, dvs)
    torch.cuda.synchronize()
    O.append(k_src, v_src, O.DTYPE_F32, hk, hv, dt, table, None, hks, hvs)
    assert np.array_equal(dk.cpu().numpy().view(np.uint8), hk.view(np.uint8)), "K codes differ"
    assert np.array_equal(dv.cpu().numpy().view(np.uint8), hv.view(np.uint8)), "V codes differ"
    if cache == "i8":
        assert np.array_equal(dks.cpu().numpy().view(np.uint32), hks.view(np.uint32)), "K scales differ"
        assert np.array_equal(dvs.cpu().numpy().view(np.uint32), hvs.view(np.uint32)), "V scales differ"


def test_fp8_codes_midpoints_and_specials(ff, gpu):
    rng = np.random.default_rng(8)
    codes = O.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    mags = np.unique(np.abs(codes[np.isfinite(codes)]))
    mids = ((mags[1:] + mags[:-1]) / 2).astype(np.float32)
    for s in (np.float32(1.0), np.float32(0.0371), np.float32(3.3e-5)):
        base = np.concatenate([mags, mids, -mags, -mids]).astype(np.float32) * s
        special = np.array([448 * s, 464 * s, 480 * s, 1e4 * s, 3.0e38, -3.0e38, np.inf, -np.inf, np.nan, 0.0, -0.0,
                            2.0 ** -10 * s, 2.0 ** -11 * s, 1e-30], np.float32)
        vals = np.concatenate([_neighbours(base.astype(np.float32)), special])
        rows = _rows(vals, rng)
        _run(ff, gpu, rows, rows[::-1].copy(), "fp8", head_scale=(s, s))


def test_int8_half_integers_and_specials(ff, gpu):
    rng = np.random.default_rng(9)
    rows = []
    for amax in (127.0, 100.0, 0.0123, 3.7e5):
        s = np.float32(np.float32(amax) / np.float32(127.0))
        half = (np.arange(-127, 127, dtype=np.float32) + np.float32(0.5))
        near = _neighbours((half * s).astype(np.float32))
        ints = (np.arange(-127, 128, dtype=np.float32) * s).astype(np.float32)
        vals = np.concatenate([near, ints])
        vals = vals[np.abs(vals) <= np.float32(amax)]
        r = _rows(vals, rng)
        r[:, 0] = np.float32(amax)  # every row's absmax is amax, so its scale is s
        rows.append(r)
    specials = np.zeros((3, D), np.float32)
    specials[0, :4] = [np.nan, 1.0, -1.0, 0.5]   # NaN ignored by the absmax, codes 0
    specials[1, :] = -0.0                        # all-zero row: scale 0, codes 0
    specials[2, :3] = [np.inf, 1.0, -2.0]        # infinite absmax
    rows = np.concatenate(rows + [specials]).astype(np.float32)
    _run(ff, gpu, rows, rows[::-1].copy(), "i8")
