"""Pins the f32 arithmetic of the oracle's dequantizers on values where
rounding shows.

The reference dequantizers (engine/core/combs-formats/src/gguf.rs) compute
  Q4_K / Q5_K  (d*sc)*q - dmin*m          (gguf.rs:906-914, 948-956)
  Q6_K         (d*sc)*q, left to right    (gguf.rs:984-987)
  Q4_1 / Q5_1  q*d + m                    (gguf.rs:812-815, 865-866)
  Q4_0 / Q5_0 / Q8_0   q*d                (gguf.rs:766-769, 838-841, 786-789)
with f32 operands: d, dmin, m converted exactly from f16 (11 significant
bits), sc and m 6-bit (Q6_K: i8, at most 7 magnitude bits), q at most 6
bits.  Every product above is therefore exact in f32 (at most
11 + 6 + 5 = 22 significant bits for the K-quants, 11 + 7 + 6 = 24 for
Q6_K's d*sc*q).  The only rounding is the final subtraction (Q4_K/Q5_K) or
addition (Q4_1/Q5_1); Q6_K never rounds.  Contracting the last step into an
FMA gives the same bits, and so does reassociating the products, with one
exception that the tests pin: the sign of a zero.  Q6_K's (d*sc)*q carries
sign(d)*sign(sc)*sign(q) when sc or q is 0 while d*(sc*q) carries sign(d), so the reference's
left-to-right order is visible in the bits of every zero it yields.

What can change the bits, and what these tests catch:
  * no rounding at all (a float64 result),
  * an intermediate rounded to fp16 (e.g. d*sc held as an fp16 scale),
  * a different decomposition (e.g. d*(sc*q - (dmin/d)*m)),
  * a wrong field, bit position, sign or bias.
Expected values are computed here with numpy float32 operations in the
reference's order, from a bit-field decoder written independently of
oracle/gguf_oracle.c; d, dmin and the scales are random non-power-of-two
values so the final operation rounds on a large share of the outputs.
"""
import numpy as np
import pytest

import oracle as O

NB = 4000  # blocks per format


def _rand_f16(rng, n, lo=-6, hi=2):
    """Random normal fp16 values 2^e * (1 + f), f with random low mantissa
    bits (never a power of two), sign random."""
    e = rng.integers(lo, hi, n).astype(np.float64)
    mant = 1.0 + (rng.integers(1, 1024, n) / 1024.0)
    s = np.where(rng.random(n) < 0.5, -1.0, 1.0)
    return (s * mant * 2.0 ** e).astype(np.float16)


def _f32(a):
    return np.asarray(a, np.float32)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _unpack_k4(scales):
    """8 six-bit scales and mins from [nb, 12] bytes: sub-blocks 0-3 take the
    low 6 bits of bytes 0-3 (scales) / 4-7 (mins); sub-blocks 4-7 take the
    nibbles of bytes 8-11 (scale low, min high) with the top two bits of
    bytes 0-3 / 4-7 above them."""
    q = scales.astype(np.int64)
    sc = np.zeros((q.shape[0], 8), np.int64)
    mn = np.zeros_like(sc)
    sc[:, :4] = q[:, 0:4] & 63
    mn[:, :4] = q[:, 4:8] & 63
    sc[:, 4:] = (q[:, 8:12] & 15) | ((q[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    return sc, mn


def _kq_blocks(rng, fmt):
    """d random; dmin 2^-4 .. 2^-10 of |d| so that (d*sc)*q and dmin*m
    overlap by only part of their bits and the difference rounds."""
    bb = {O.Q4_K: 144, O.Q5_K: 176}[fmt]
    blk = rng.integers(0, 256, (NB, bb), dtype=np.uint8)
    d = _rand_f16(rng, NB)
    dmin = (np.abs(d).astype(np.float64) * 2.0 ** -rng.integers(4, 11, NB)
            * (1.0 + rng.integers(1, 1024, NB) / 1024.0)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(NB, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(NB, 2)
    return blk


def _expect_kq(blk, fmt):
    """(d*sc)*q - dmin*m in f32, value order of gguf.rs:894-961."""
    nb = blk.shape[0]
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb)
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nb)
    sc, mn = _unpack_k4(blk[:, 4:16])
    qs = blk[:, -128:].astype(np.int64).reshape(nb, 4, 32)  # group j, byte l
    q = np.zeros((nb, 8, 32), np.int64)  # sub-block 2j: low nibbles, 2j+1: high
    q[:, 0::2] = qs & 15
    q[:, 1::2] = qs >> 4
    if fmt == O.Q5_K:
        qh = blk[:, 16:48].astype(np.int64)  # [nb, 32], bit 2j+t of qh[l]
        for s in range(8):
            q[:, s] |= ((qh >> s) & 1) << 4
    d1 = _f32(d[:, None] * _f32(sc))            # exact
    fm = _f32(dmin[:, None] * _f32(mn))          # exact
    v = _f32(_f32(d1[:, :, None] * _f32(q)) - fm[:, :, None])
    return v.reshape(nb, 256), (d, dmin, sc, mn, q)


def _q6_blocks(rng):
    blk = rng.integers(0, 256, (NB, 210), dtype=np.uint8)
    blk[:, 208:210] = _rand_f16(rng, NB).view(np.uint8).reshape(NB, 2)
    return blk


def _expect_q6(blk):
    """d * sc * q left to right (gguf.rs:968-999)."""
    nb = blk.shape[0]
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32).reshape(nb)
    out = np.zeros((nb, 256), np.float32)
    qq = np.zeros((nb, 256), np.int64)
    ss = np.zeros((nb, 256), np.int64)
    for h in range(2):
        ql = blk[:, 64 * h:64 * h + 64].astype(np.int64)
        qh = blk[:, 128 + 32 * h:160 + 32 * h].astype(np.int64)
        sc = blk[:, 192 + 8 * h:200 + 8 * h].view(np.int8).astype(np.int64)
        for t in range(4):  # quadrant t: ql[l + 32*(t&1)], nibble t>>1, qh bits 2t
            lo = ql[:, 32 * (t & 1):32 * (t & 1) + 32]
            nib = (lo >> (4 * (t >> 1))) & 15
            q = (nib | (((qh >> (2 * t)) & 3) << 4)) - 32
            s = np.repeat(sc[:, [2 * t, 2 * t + 1]], 16, axis=1)
            i0 = 128 * h + 32 * t
            qq[:, i0:i0 + 32] = q
            ss[:, i0:i0 + 32] = s
    out[:] = _f32(_f32(d[:, None] * _f32(ss)) * _f32(qq))
    return out, (d, ss, qq)


def _q51_blocks(rng, fmt):
    bb = 24 if fmt == O.Q5_1 else 20
    blk = rng.integers(0, 256, (NB, bb), dtype=np.uint8)
    d = np.abs(_rand_f16(rng, NB, -14, -10))
    m = _rand_f16(rng, NB, 4, 10)  # m 2^14 .. 2^24 times d: q*d + m rounds
    blk[:, 0:2] = d.view(np.uint8).reshape(NB, 2)
    blk[:, 2:4] = m.view(np.uint8).reshape(NB, 2)
    return blk


def _expect_q51(blk, fmt):
    """q*d + m (gguf.rs:798-874): low nibbles -> values 0..15, high -> 16..31,
    Q5_1's qh bit j / j+16 as the 5th bit."""
    nb = blk.shape[0]
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb)
    m = blk[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nb)
    qs = blk[:, -16:].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    if fmt == O.Q5_1:
        qh = blk[:, 4:8].copy().view(np.uint32).astype(np.int64).reshape(nb)
        q |= ((qh[:, None] >> np.arange(32)) & 1) << 4
    return _f32(_f32(_f32(q) * d[:, None]) + m[:, None]), (d, m, q)


def _dq(fmt, blk):
    return O.dequant(fmt, blk.tobytes(), blk.shape[0] * O.block_values(fmt)).reshape(blk.shape[0], -1)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q5_K])
def test_kquant_rounding_bits(fmt):
    rng = np.random.default_rng(40 + fmt)
    blk = _kq_blocks(rng, fmt)
    want, (d, dmin, sc, mn, q) = _expect_kq(blk, fmt)
    got = _dq(fmt, blk)
    assert np.array_equal(_bits(got), _bits(want))
    # the subtraction rounds on a large share of outputs: an exact (float64)
    # evaluation, or a float32 evaluation that skipped the rounding, differs
    exact = (d[:, None, None].astype(np.float64) * sc[:, :, None] * q
             - dmin[:, None, None].astype(np.float64) * mn[:, :, None]).reshape(-1, 256)
    frac_rounded = np.mean(exact != want.astype(np.float64))
    assert frac_rounded > 0.2, frac_rounded
    # holding d*sc as an fp16 scale changes many values
    d1h = (d[:, None] * sc).astype(np.float16).astype(np.float32)
    alt = _f32(_f32(d1h[:, :, None] * _f32(q)) - _f32(dmin[:, None] * _f32(mn))[:, :, None]).reshape(-1, 256)
    assert np.mean(alt != want) > 0.1
    # another decomposition: d * (sc*q - (dmin/d)*m)
    alt2 = _f32(d[:, None, None] * _f32(_f32(sc[:, :, None] * q) - _f32(dmin / d)[:, None, None] * _f32(mn)[:, :, None]))
    assert np.mean(alt2.reshape(-1, 256) != want) > 0.1


def test_q6_k_rounding_bits():
    rng = np.random.default_rng(46)
    blk = _q6_blocks(rng)
    want, (d, ss, qq) = _expect_q6(blk)
    got = _dq(O.Q6_K, blk)
    assert np.array_equal(_bits(got), _bits(want))
    # every product is exact ...
    exact = d[:, None].astype(np.float64) * ss * qq
    assert np.array_equal(exact, want.astype(np.float64))
    # ... and a zero carries sign(d) * sign(sc) (left-to-right (d*sc)*q)
    z = qq == 0
    assert z.sum() > 1000
    neg = (np.signbit(d)[:, None] != (ss < 0))
    assert np.array_equal(np.signbit(want)[z], neg[z])
    # d*(sc*q) gives those zeros sign(d) instead: its bits differ
    alt = _f32(d[:, None] * _f32(ss * qq))
    assert np.any(_bits(alt) != _bits(want))
    # holding d*sc as an fp16 scale changes many values
    alt = _f32((d[:, None] * ss).astype(np.float16).astype(np.float32) * _f32(qq))
    assert np.mean(alt != want) > 0.1


@pytest.mark.parametrize("fmt", [O.Q4_1, O.Q5_1])
def test_affine_legacy_rounding_bits(fmt):
    rng = np.random.default_rng(50 + fmt)
    blk = _q51_blocks(rng, fmt)
    want, (d, m, q) = _expect_q51(blk, fmt)
    got = _dq(fmt, blk)
    assert np.array_equal(_bits(got), _bits(want))
    exact = q * d[:, None].astype(np.float64) + m[:, None].astype(np.float64)
    assert np.mean(exact != want.astype(np.float64)) > 0.3
    # adding m before scaling (q + m/d) * d rounds differently
    alt = _f32(_f32(_f32(q) + _f32(m / d)[:, None]) * d[:, None])
    assert np.mean(alt != want) > 0.1


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q5_0, O.Q8_0])
def test_symmetric_legacy_bits(fmt):
    """One f32 product of exact operands: equal to the exactly rounded
    d*q (checked against float64, where the product is exact)."""
    rng = np.random.default_rng(60 + fmt)
    bb = O.block_bytes(fmt)
    blk = rng.integers(0, 256, (NB, bb), dtype=np.uint8)
    blk[:, 0:2] = _rand_f16(rng, NB).view(np.uint8).reshape(NB, 2)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(NB)
    if fmt == O.Q8_0:
        q = blk[:, 2:].view(np.int8).astype(np.int64)
    else:
        qs = blk[:, -16:].astype(np.int64)
        q = np.concatenate([qs & 15, qs >> 4], axis=1)
        if fmt == O.Q5_0:
            qh = blk[:, 2:6].copy().view(np.uint32).astype(np.int64).reshape(NB)
            q = (q | (((qh[:, None] >> np.arange(32)) & 1) << 4)) - 16
        else:
            q = q - 8
    want = (q * d[:, None]).astype(np.float32)  # exact in float64, one rounding
    assert np.array_equal(_bits(_dq(fmt, blk)), _bits(want))


def test_products_exact_so_order_is_fixed():
    """Why 'separately rounded' versus 'FMA-contracted' or 'd*(sc*q)' cannot
    differ: the products are exact in f32, so every order rounds the same
    real number once.  Checked on the random blocks above by evaluating the
    FMA form (exact float64 product and difference, one rounding to f32)."""
    rng = np.random.default_rng(41)
    for fmt in (O.Q4_K, O.Q5_K):
        blk = _kq_blocks(rng, fmt)
        want, (d, dmin, sc, mn, q) = _expect_kq(blk, fmt)
        d1 = (d[:, None] * sc).astype(np.float64)
        assert np.array_equal(d1, (d[:, None].astype(np.float64) * sc))  # d*sc exact
        fma = (d1[:, :, None] * q - (dmin[:, None].astype(np.float64) * mn)[:, :, None]).astype(np.float32)
        assert np.array_equal(_bits(fma.reshape(-1, 256)), _bits(want))
        reassoc = _f32(d[:, None, None] * _f32(sc[:, :, None] * q)) - _f32(dmin[:, None] * _f32(mn))[:, :, None]
        assert np.array_equal(_bits(_f32(reassoc).reshape(-1, 256)), _bits(want))
    blk = _q6_blocks(rng)
    want, (d, ss, qq) = _expect_q6(blk)
    nz = ss * qq != 0  # reassociation agrees except for the sign of zeros
    alt = _f32(d[:, None] * _f32(ss * qq))
    assert np.array_equal(_bits(alt)[nz], _bits(want)[nz])
