"""The int8 quantiser's no-division fast path, emulated on the CPU.

The device kernels (quant_rows_i8_*_kernel / quant8) does not divide each
element by the row scale s = absmax / 127.  It forms the biased code
u = fma(x, 1/s, 128), rounds it, and redoes a chunk with the division only
when some element lies near a half-integer.  That shortcut is exact only
while 1/s is a finite reciprocal: for a row whose absmax is below about
127 * 2^-128 (3.7e-37), s is a tiny subnormal and 1/s overflows to +inf.

These tests restate the device arithmetic in numpy float32 (the fma as an
exact float64 product plus 128, rounded once to float32 -- exact here,
since |x * inv| <= 128 needs at most 48 bits) and check both the old
redo predicate, which misses that case, and the current one, against the
oracle's division (oracle.quant_rows_i8)."""
import numpy as np
import pytest

import oracle

LIMIT = np.float32(0.5) - np.float32(5e-5)
FLT_MAX = np.float32(3.4028234663852886e38)


def _cvt_pk_u8(n):
    """v_cvt_pk_u8_f32: float -> unsigned byte, saturating; NaN -> 0."""
    out = np.where(np.isnan(n), 0.0, np.clip(n, 0.0, 255.0))
    return out.astype(np.uint8)


def _division_codes(x, s):
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        t = x / s
    r = np.sign(t) * np.floor(np.abs(t) + np.float32(0.5))     # half away
    r = np.where(np.isnan(r), -127.0, r)                       # fmaxf drops NaN
    return np.clip(r, -127, 127).astype(np.int8)


def emulate_row(xbits, new_predicate):
    """The device's codes for one bf16 row, chunk by chunk (8 elements)."""
    x = oracle.bf16_to_f32(xbits).astype(np.float32)
    amax = np.float32(np.max(np.abs(x)))
    s = np.float32(amax / np.float32(127.0))
    if s == 0:
        return np.zeros(x.size, np.int8), s
    with np.errstate(divide="ignore", over="ignore"):
        inv = np.float32(np.float32(1.0) / s)
    fast = bool(inv <= FLT_MAX)
    codes = np.empty(x.size, np.int8)
    for c0 in range(0, x.size, 8):
        xc = x[c0:c0 + 8]
        with np.errstate(invalid="ignore", over="ignore"):
            u = (xc.astype(np.float64) * np.float64(inv) + 128.0).astype(np.float32)
            n = np.rint(u)
            d = np.abs(u - n)
        if new_predicate:
            redo = (not fast) or bool(np.any(~(d <= LIMIT)))
        else:
            dev = np.float32(0.0)
            for v in d:
                dev = np.fmax(dev, v)          # fmaxf: a NaN operand is dropped
            redo = bool(dev > LIMIT)
        if redo:
            codes[c0:c0 + 8] = _division_codes(xc, s)
        else:
            codes[c0:c0 + 8] = (_cvt_pk_u8(n) ^ np.uint8(0x80)).view(np.int8)
    return codes, s


def _row(values, K=64):
    row = np.zeros(K, np.float32)
    row[:len(values)] = values
    return oracle.f32_to_bf16(row[None, :])[0]


TINY_ROWS = {
    "absmax 1e-37": [1e-37, 5e-38, 0.0, -2e-38, 3.3e-38, -1e-37],
    "absmax 1e-38": [1e-38, -7e-39, 2e-39],
    "smallest bf16 subnormal": [np.float32(2.0 ** -133), -np.float32(2.0 ** -133)],
    "smallest bf16 normal": [np.float32(2.0 ** -126), np.float32(2.0 ** -127)],
}


@pytest.mark.parametrize("name", sorted(TINY_ROWS))
def test_old_predicate_misses_overflowing_reciprocal(name):
    """With 1/s = +inf every product is +-inf or NaN; the old predicate
    (fmaxf of the deviations, then `>`) never redoes the chunk, and the
    packed codes are not the division's."""
    xb = _row(TINY_ROWS[name])
    qo, so = oracle.quant_rows_i8(xb[None, :])
    x = oracle.bf16_to_f32(xb)
    s = np.float32(np.max(np.abs(x)) / np.float32(127.0))
    with np.errstate(divide="ignore", over="ignore"):
        assert not np.isfinite(np.float32(1.0) / s)        # the case at hand
    old, s_old = emulate_row(xb, new_predicate=False)
    assert s_old.view(np.uint32) == so[0].view(np.uint32)
    assert not np.array_equal(old, qo[0])


@pytest.mark.parametrize("name", sorted(TINY_ROWS))
def test_current_predicate_matches_division(name):
    xb = _row(TINY_ROWS[name])
    qo, _ = oracle.quant_rows_i8(xb[None, :])
    new, _ = emulate_row(xb, new_predicate=True)
    assert np.array_equal(new, qo[0])
    assert new.min() >= -127


def test_subnormal_scale_with_finite_reciprocal():
    """absmax 1e-36: s is subnormal but 1/s is finite, so the fast path runs
    and still gives the division's codes (with random elements)."""
    rng = np.random.default_rng(5)
    vals = rng.uniform(-1e-36, 1e-36, 64).astype(np.float32)
    vals[3] = 1e-36
    xb = _row(vals)
    x = oracle.bf16_to_f32(xb)
    s = np.float32(np.max(np.abs(x)) / np.float32(127.0))
    assert s < np.finfo(np.float32).tiny                     # subnormal
    assert np.isfinite(np.float32(1.0) / s)
    qo, _ = oracle.quant_rows_i8(xb[None, :])
    for pred in (False, True):
        got, _ = emulate_row(xb, new_predicate=pred)
        assert np.array_equal(got, qo[0])


def test_ordinary_rows_agree_either_way():
    """On ordinary rows (absmax ~1) both predicates give the division's
    codes: the fast path's error bound holds."""
    rng = np.random.default_rng(6)
    xb = oracle.f32_to_bf16(rng.standard_normal((8, 256)).astype(np.float32))
    qo, _ = oracle.quant_rows_i8(xb)
    for r in range(xb.shape[0]):
        for pred in (False, True):
            got, _ = emulate_row(xb[r], new_predicate=pred)
            assert np.array_equal(got, qo[r])
