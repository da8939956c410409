"""The host quantisers (input generation).  Q8_0 and Q4_0 follow the rules
BASELINE states exactly (d = max|x|/127, q = round(x/d); d = max/-8,
q = x/d + 8 clamped to 15), checked byte for byte against a numpy
restatement; the K-quants (ggml's iterative fits) are checked by round-trip
error bounds and field validity.  Bit equality with ggml's own output is not
pinned: ggml is not available here."""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat, quantize

RNG = np.random.default_rng(1234)


def _np_q8_0(x):
    out = bytearray()
    for blk in x.reshape(-1, 32):
        amax = np.float32(np.max(np.abs(blk)))
        d = np.float32(amax / np.float32(127))
        idv = np.float32(1) / d if d else np.float32(0)
        q = np.trunc(blk * idv + np.copysign(np.float32(0.5), blk * idv))  # roundf: half away from 0
        out += np.float16(d).tobytes() + q.astype(np.int8).tobytes()
    return bytes(out)


def _np_q4_0(x):
    out = bytearray()
    for blk in x.reshape(-1, 32):
        i = int(np.argmax(np.abs(blk)))
        mx = blk[i]
        d = np.float32(mx / np.float32(-8))
        idv = np.float32(1) / d if d else np.float32(0)
        q = np.minimum(15, np.trunc(blk * idv + np.float32(8.5)).astype(np.int32))
        out += np.float16(d).tobytes() + bytes((q[:16] | (q[16:] << 4)).astype(np.uint8))
    return bytes(out)


def test_q8_0_matches_rule():
    x = RNG.normal(0, 0.02, (8, 576)).astype(np.float32)
    assert quantize(QuantFormat.Q8_0, x) == _np_q8_0(x)


def test_q4_0_matches_rule():
    x = RNG.normal(0, 0.02, (8, 512)).astype(np.float32)
    assert quantize(QuantFormat.Q4_0, x) == _np_q4_0(x)


# |error| / max|x| per block.  Q4_0/Q5_0: the side opposite the max clamps at
# 7d / 15d, so up to one step (1/8, 1/16 of max|x|); Q8_0: half a step plus the
# f16 rounding of d.  K-quant bounds are loose empirical envelopes.
BOUND = {QuantFormat.Q4_0: 1 / 8 + 1e-3, QuantFormat.Q5_0: 1 / 16 + 1e-3, QuantFormat.Q8_0: 1 / 200,
         QuantFormat.Q4_1: 1 / 15 + 1e-3, QuantFormat.Q5_1: 1 / 31 + 1e-3,
         QuantFormat.Q4K: 1 / 8, QuantFormat.Q5K: 1 / 16, QuantFormat.Q6K: 1 / 40}


@pytest.mark.parametrize("fmt", list(QuantFormat))
def test_round_trip_error(fmt):
    x = RNG.normal(0, 0.02, (16, 1024)).astype(np.float32)
    b = quantize(fmt, x)
    w = O.dequant(int(fmt), b, x.size).reshape(x.shape)
    qk = O.block_values(int(fmt))
    err = np.abs(w - x).reshape(-1, qk).max(1)
    amax = np.abs(x).reshape(-1, qk).max(1)
    assert np.all(err <= BOUND[fmt] * amax + 1e-7)
    # and it is a real fit, not zeros
    assert np.abs(w).max() > 0.5 * np.abs(x).max()


def test_k_quant_fields_valid():
    x = RNG.normal(0, 0.02, (4, 512)).astype(np.float32)
    b = np.frombuffer(quantize(QuantFormat.Q4K, x), np.uint8).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(d)) and np.all(d > 0)
    b6 = np.frombuffer(quantize(QuantFormat.Q6K, x), np.uint8).reshape(-1, 210)
    sc = b6[:, 192:208].view(np.int8)
    assert sc.min() >= -128 and sc.max() <= 127
    assert (np.abs(sc.astype(np.int32)).max(1) >= 100).all()  # scales span the i8 range


def test_zero_input():
    for fmt in QuantFormat:
        x = np.zeros((1, 256), np.float32)
        b = quantize(fmt, x)
        assert np.all(O.dequant(int(fmt), b, 256) == 0)
