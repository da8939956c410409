"""Pins the CPU oracle (oracle/gguf_oracle.c) before anything is compared
against it: reference known answers, exhaustive f16 conversion, single-field
position probes derived from the GGUF layout, scale_min_k4 against an
independent packer, and the reference matmul against float64."""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")


def test_f16_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("fmt,n,k,expect", [
    # gguf.rs:732-740 block sizes at the benchmark shapes
    (O.Q4_K, 14336, 4096, 33030144), (O.Q6_K, 128256, 4096, 430940160),
    (O.Q8_0, 1536, 576, 940032), (O.Q4_0, 4096, 4096, 9437184), (O.Q5_K, 14336, 4096, 40370176),
    (O.Q8_0, 4096, 14336, 62390272),
])
def test_tensor_bytes(fmt, n, k, expect):
    assert O.tensor_bytes(fmt, n * k) == expect


def test_tensor_bytes_rejects_ragged():
    assert O.tensor_bytes(O.Q4_K, 128) == -1
    assert O.tensor_bytes(O.Q4_0, 31) == -1


@pytest.mark.parametrize("name", ["q8_0_gguf_roundtrip", "q4_0_reference_block", "q4_0_all_eights"])
def test_reference_known_answers(name):
    case = json.load(open(GOLD))[name]
    got = O.dequant(case["format"], bytes.fromhex(case["hex"]), case["n"])
    assert np.array_equal(got, np.array(case["expect"], np.float32))


def _f16(v):
    return np.array([v], np.float16).tobytes()


def _probe(fmt, base: bytearray, byte: int, val: int):
    b = bytearray(base)
    b[byte] = val
    return O.dequant(fmt, bytes(b), O.block_values(fmt))


def test_q4_0_positions():
    base = bytearray(_f16(1.0) + bytes([0x88] * 16))
    for j in range(16):
        v = _probe(O.Q4_0, base, 2 + j, 0x8B)  # low nibble 11 -> +3 at j
        e = np.zeros(32, np.float32)
        e[j] = 3
        assert np.array_equal(v, e)
        v = _probe(O.Q4_0, base, 2 + j, 0xB8)  # high nibble -> +3 at j+16
        e = np.zeros(32, np.float32)
        e[j + 16] = 3
        assert np.array_equal(v, e)


def test_q5_0_positions():
    # d = 1, nibbles 0, qh = 0 -> every value -16; set qh bit i -> value i is 0.
    for i in range(32):
        qh = (1 << i).to_bytes(4, "little")
        v = O.dequant(O.Q5_0, _f16(1.0) + qh + bytes(16), 32)
        e = np.full(32, -16.0, np.float32)
        e[i] = 0.0
        assert np.array_equal(v, e)


def test_q4_1_positions_and_min():
    # gguf.rs:798-820: value = q * d + m; d = 0.5, m = -2: low nibble j -> value
    # j, high nibble -> j + 16; q = 0 gives m exactly.
    for j in range(16):
        q = bytearray(16)
        q[j] = 0x3C  # low 12, high 3
        v = O.dequant(O.Q4_1, _f16(0.5) + _f16(-2.0) + bytes(q), 32)
        e = np.full(32, -2.0, np.float32)
        e[j] = 12 * 0.5 - 2.0
        e[j + 16] = 3 * 0.5 - 2.0
        assert np.array_equal(v, e)


def test_q5_1_positions_and_min():
    # gguf.rs:851-874: qh bit i is the 5th bit of value i; d = 1, m = 0.25
    for i in range(32):
        qh = (1 << i).to_bytes(4, "little")
        v = O.dequant(O.Q5_1, _f16(1.0) + _f16(0.25) + qh + bytes([0x21] * 16), 32)
        e = np.array([1.25] * 16 + [2.25] * 16, np.float32)
        e[i] += 16.0
        assert np.array_equal(v, e)


def test_q4_1_rounding_order():
    # q * d rounded, then + m rounded (two f32 roundings, no fused multiply-add):
    # d = 1 + 2^-10, q = 15, m = 2^-13 -> 15 * d is exact, + m rounds.
    d, m = np.float16(1 + 2 ** -10), np.float16(2 ** -13)
    v = O.dequant(O.Q4_1, d.tobytes() + m.tobytes() + bytes([0x0F] + [0] * 15), 32)
    assert v[0] == np.float32(np.float32(15) * np.float32(d)) + np.float32(m)


def test_q8_0_positions_and_sign():
    for j in range(32):
        q = bytearray(32)
        q[j] = 0x81  # -127
        v = O.dequant(O.Q8_0, _f16(0.5) + bytes(q), 32)
        e = np.zeros(32, np.float32)
        e[j] = -63.5
        assert np.array_equal(v, e)


# K-quant superblocks with d = 1, dmin = 0 and every 6-bit scale = 1, min = 0.
UNIT_SCALES = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])


def test_q4_k_positions():
    base = bytearray(_f16(1.0) + _f16(0.0) + UNIT_SCALES + bytes(128))
    for b in range(128):
        j, l = divmod(b, 32)  # gguf.rs:903-915: group j, low nibble -> 64j+l, high -> 64j+32+l
        v = _probe(O.Q4_K, base, 16 + b, 0x21)
        e = np.zeros(256, np.float32)
        e[64 * j + l] = 1
        e[64 * j + 32 + l] = 2
        assert np.array_equal(v, e), b


def test_q5_k_positions():
    base = bytearray(_f16(1.0) + _f16(0.0) + UNIT_SCALES + bytes(32) + bytes(128))
    for l in range(32):
        for bit in range(8):  # qh[l] bit 2j+t -> value 64j + 32t + l gets +16
            v = _probe(O.Q5_K, base, 16 + l, 1 << bit)
            j, t = divmod(bit, 2)
            e = np.zeros(256, np.float32)
            e[64 * j + 32 * t + l] = 16
            assert np.array_equal(v, e)
    for b in range(128):
        j, l = divmod(b, 32)
        v = _probe(O.Q5_K, base, 48 + b, 0x21)
        e = np.zeros(256, np.float32)
        e[64 * j + l] = 1
        e[64 * j + 32 + l] = 2
        assert np.array_equal(v, e)


def _q6_index(h, t, l):
    return 128 * h + 32 * t + l


def test_q6_k_positions():
    # d = 1, all 16 scales 1, ql = qh = 0 -> every value is -32.
    base = bytearray(bytes(192) + bytes([1] * 16) + _f16(1.0))
    flat = np.full(256, -32.0, np.float32)
    for h in range(2):
        for b in range(64):  # ql[64h + b]: b<32 -> quadrants 0 (lo) / 2 (hi); b>=32 -> 1 / 3
            u, l = divmod(b, 32)
            v = _probe(O.Q6_K, base, 64 * h + b, 0x52)  # lo nibble 2, hi nibble 5
            e = flat.copy()
            e[_q6_index(h, u, l)] = 2 - 32
            e[_q6_index(h, u + 2, l)] = 5 - 32
            assert np.array_equal(v, e)
        for l in range(32):  # qh[32h + l] bits 2t..2t+1 -> quadrant t, +16 per unit
            v = _probe(O.Q6_K, base, 128 + 32 * h + l, 0b11100100)  # t0:0 t1:1 t2:2 t3:3
            e = flat.copy()
            for t in range(4):
                e[_q6_index(h, t, l)] = 16 * t - 32
            assert np.array_equal(v, e)
        for s in range(8):  # scale 8h + s covers l in [16*(s%2), +16) of quadrant s//2
            v = _probe(O.Q6_K, base, 192 + 8 * h + s, 3)
            e = flat.copy()
            t, half = divmod(s, 2)
            for l in range(16 * half, 16 * half + 16):
                e[_q6_index(h, t, l)] = -96
            assert np.array_equal(v, e)


def _pack_scales_k4(sc, mn):
    """Independent packer: ggml's layout of 8 6-bit scales + 8 6-bit mins in
    12 bytes, written from the bit-field description (not from the unpacker)."""
    q = [0] * 12
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(q)


def test_scale_min_k4_against_packer():
    rng = np.random.default_rng(1)
    for trial in range(2000):
        sc = rng.integers(0, 64, 8).tolist()
        mn = rng.integers(0, 64, 8).tolist()
        if trial < 64:  # every value in every slot at least once
            sc = [(trial + j) % 64 for j in range(8)]
            mn = [(3 * trial + j) % 64 for j in range(8)]
        packed = _pack_scales_k4(sc, mn)
        for j in range(8):
            assert O.scale_min_k4(j, packed) == (sc[j], mn[j])


def test_q4_k_closed_form_constant_block():
    # all nibbles q, all scales s, all mins m: value = (d*s)*q - dmin*m exactly
    for q in (0, 7, 15):
        for s, m in ((1, 0), (63, 63), (17, 5)):
            packed = _pack_scales_k4([s] * 8, [m] * 8)
            blk = _f16(0.25) + _f16(0.125) + packed + bytes([q | (q << 4)] * 128)
            v = O.dequant(O.Q4_K, blk, 256)
            want = np.float32(np.float32(0.25) * np.float32(s)) * np.float32(q) - np.float32(np.float32(0.125) * np.float32(m))
            assert np.all(v == want)


def test_ref_matmul_vs_float64():
    rng = np.random.default_rng(2)
    x = rng.normal(size=(3, 257)).astype(np.float32)
    w = rng.normal(size=(19, 257)).astype(np.float32)
    got = O.ref_matmul(x, w).astype(np.float64)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 257 * np.finfo(np.float32).eps * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got - exact) <= bound)
    # a transposed operand or dropped term would be far outside the bound
    assert not np.allclose(O.ref_matmul(x, w[::-1].copy()), got)


@pytest.mark.parametrize("fmt,n,k", [(O.Q4_0, 67, 128), (O.Q5_0, 67, 128), (O.Q8_0, 67, 128),
                                     (O.Q4_K, 35, 512), (O.Q5_K, 35, 512), (O.Q6_K, 35, 512)])
def test_fused_matches_ref_matmul(fmt, n, k):
    """The reference's fused accumulation order vs ref_matmul over the
    dequant, at the reference's own tolerance (qmatmul.rs:1751-1781, 1893-1971)."""
    data = O.SYNTH[fmt](n * k // O.block_values(fmt))
    w = O.dequant(fmt, data, n * k).reshape(n, k)
    for m in (1, 3):
        x = O.x_pattern(m, k).reshape(m, k)
        O.assert_close(O.fused_matmul(fmt, data, x, n, k), O.ref_matmul(x, w),
                       1e-4 if fmt == O.Q4_0 else 1e-3, f"fmt{fmt} m={m}")


def test_synth_streams_have_reference_shape():
    assert len(O.synth_q4_0(33)) == 33 * 18
    assert len(O.synth_q4_k(9)) == 9 * 144
    assert len(O.synth_q6_k(9)) == 9 * 210
    # synth_q6_k stores d last (qmatmul.rs:1821-1829): f16(0.002) for b=0
    assert O.synth_q6_k(1)[208:210] == _f16(np.float32(0.002))
    # one running LCG across blocks for Q4_0 (qmatmul.rs:1700-1708)
    a = O.synth_q4_0(2)
    assert a[2:18] == O.lcg_bytes(16, 0x12345678)


def test_dense_gemm_matches_ref():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 576)).astype(np.float32)
    w = rng.normal(size=(40, 576)).astype(np.float32)
    O.assert_close(O.dense_gemm(x, w, 1), O.ref_matmul(x, w), 1e-4)
    O.assert_close(O.dense_gemm(x, w, 4), O.ref_matmul(x, w), 1e-4)


def test_activation_gelu_tanh_known_values():
    # act.rs:41-52: torch gelu(approximate="tanh") at -1, 0, 1, 2
    got = O.activation(O.ACT_GELU_TANH, [-1.0, 0.0, 1.0, 2.0])
    assert np.all(np.abs(got - [-0.158808, 0.0, 0.841192, 1.954597]) < 1e-5)


def test_activation_silu_identities():
    v = np.linspace(-30, 30, 1201)
    s = O.activation(O.ACT_SILU, v)
    assert O.activation(O.ACT_SILU, [0.0])[0] == 0.0
    # x*sigmoid(x) - (-x)*sigmoid(-x) = x (sigmoid(x) + sigmoid(-x) = 1)
    assert np.allclose(s - O.activation(O.ACT_SILU, -v), v, rtol=0, atol=1e-12)
    # sigmoid(x) -> 1 and -> 0 at the ends; sigmoid(1) = e / (1 + e)
    assert abs(s[-1] - 30.0) < 1e-11 and abs(s[0]) < 1e-11
    assert abs(O.activation(O.ACT_SILU, [1.0])[0] - np.e / (1 + np.e)) < 1e-15


def test_activation_gelu_is_x_times_normal_cdf():
    # Phi(1) = 0.8413447460685429, Phi(2) = 0.9772498680518208 (normal tables)
    got = O.activation(O.ACT_GELU, [1.0, -1.0, 2.0, 0.0])
    want = [0.8413447460685429, -(1 - 0.8413447460685429), 2 * 0.9772498680518208, 0.0]
    assert np.allclose(got, want, rtol=0, atol=1e-15)
    # tanh form approximates the exact one to < 1e-3 on [-4, 4]
    v = np.linspace(-4, 4, 801)
    assert np.max(np.abs(O.activation(O.ACT_GELU, v) - O.activation(O.ACT_GELU_TANH, v))) < 1e-3


def test_linear_bias_and_gated_up_compose_the_op():
    k, n, m = 256, 5, 2
    data = O.synth_q4_k(n)
    x = O.x_pattern(m, k).reshape(m, k)
    y = O.fused_matmul(O.Q4_K, data, x, n, k).astype(np.float64)
    b = np.arange(n) - 2.0
    assert np.array_equal(O.linear(O.Q4_K, data, x, n, k, b), y + b)
    g = O.gated_up(O.ACT_SILU, (O.Q4_K, data), (O.Q4_K, data), x, n, k)
    assert np.allclose(g, y * y / (1 + np.exp(-y)), rtol=1e-15, atol=0)
