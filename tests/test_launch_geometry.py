"""CPU bounds check of the 16-row MFMA decode GEMV's launch geometry
(cq_gemv_*, combsengine_amd/csrc/cq_gemv.h gemv_body, host side
launch_gemv in cq_host.cpp) and of the prefill GEMM's scratch layout
(launch_gemm2 / gemm2_body / cq_splitk_reduce_*).

The host arithmetic is restated here and every index each kernel forms is
enumerated -- per activation-chunk, wave, lane group and MFMA step -- for the
shapes of a benchmark run that once faulted the GPU box (decode m = 8 / 16 at
K = 3584 and 18944, several LDS chunks) and a sweep of chunk counts,
formats, fp16 / fp32 activations and ragged tiles, and checked against the
allocation each index addresses:
  * weight bytes: each lane's units stay inside its row;
  * activation reads (staging): row < M, column range inside [0, K);
  * LDS: staging stores and MFMA operand reads inside the dynamic
    allocation, and every read of chunk c falls in the part of the row that
    chunk c staged;
  * outputs: stores only for m < M, n < N;
  * split-K: partial-sum and activation-sum offsets inside the scratch the
    host allocates.
"""
import math

import numpy as np
import pytest

# format: (values per unit, bytes per unit, block values)
UNIT = {"q4_0": (128, 72, 32), "q5_0": (128, 88, 32), "q8_0": (128, 136, 32), "q4_1": (128, 80, 32),
        "q5_1": (128, 96, 32), "q4_k": (256, 144, 256), "q5_k": (256, 176, 256), "q6_k": (256, 210, 256)}
LB = 4
LDS_BUDGET = 56 * 1024
LDS_MAX = 64 * 1024
RED_BYTES = 8 * 4 * 64 * 4  # static reduction array of gemv_body


def host_geometry(fmt, M, K, xt):
    """launch_gemv (cq_host.cpp): kc, lds_stride, dynamic LDS bytes, waves."""
    vals, _, qk = UNIT[fmt]
    blocks = K // qk
    units = blocks if qk == 256 else (blocks + 3) // 4
    unit_vals = 256 if qk == 256 else 128
    mrows = min(16, M)
    xmul = 2 if xt else 1
    kc = LDS_BUDGET // (2 * xmul * mrows) - 8
    kc -= kc % unit_vals
    k_units = -(-K // unit_vals) * unit_vals
    kc = min(kc, k_units)
    stride = kc + 8
    lds = xmul * mrows * stride * 2
    nw = min(8, max(1, -(-units // 4)))
    return dict(units=units, kc=kc, stride=stride, lds=lds, nw=nw, mrows=mrows, xmul=xmul)


def check_gemv(fmt, M, N, K, xt):
    vals, ubytes, qk = UNIT[fmt]
    geo = host_geometry(fmt, M, K, xt)
    kc, stride, nw, mrows, xmul = geo["kc"], geo["stride"], geo["nw"], geo["mrows"], geo["xmul"]
    assert kc > 0 and kc % (256 if qk == 256 else 128) == 0
    assert geo["lds"] + RED_BYTES <= LDS_MAX, "LDS over the workgroup limit"
    blocks = K // qk
    row_bytes = blocks * (ubytes // (LB if qk == 32 else 1)) if qk == 32 else blocks * ubytes
    lds_halves = xmul * mrows * stride
    chunks = 0
    for by in range(-(-M // 16)):
        m0 = by * 16
        mt = min(16, M - m0)
        for c0 in range(0, K, kc):
            chunks += by == 0
            ln = min(kc, K - c0)
            u_end = -(-(c0 + ln) // vals)
            # staging: thread i (all of 64 nw threads, XS_REG rounds and the
            # remainder loop cover i < total) -> row r, vector v
            vec = ln >> 3
            assert ln % 8 == 0
            total = mt * vec
            i = np.arange(total)
            r, v = i // vec, i % vec
            assert np.all(m0 + r < M)
            col = c0 + 8 * v
            assert np.all(col >= 0) and np.all(col + 8 <= K)
            # the float-reciprocal division of div_small is exact here
            rcp = np.float32(1.0) / np.float32(vec)
            assert np.array_equal(((i.astype(np.float32) + np.float32(0.5)) * rcp).astype(np.int64), r)
            dst = r * stride + 8 * v
            assert np.all(dst + 8 <= mrows * stride)
            if xt:
                assert np.all(mrows * stride + dst + 8 <= lds_halves)
            # x byte offsets fit the kernel's 32-bit arithmetic
            assert (m0 + mt - 1) * K * (4 if xt else 2) + (K - 1) * (4 if xt else 2) < 2 ** 31
            staged = np.zeros(mrows * stride, bool)
            staged[(dst[:, None] + np.arange(8)).ravel()] = True
            for wave in range(nw):
                us = np.arange(c0 // vals + wave, u_end, nw)
                loads = np.minimum(np.arange(c0 // vals + wave, u_end + 4 * nw, nw), u_end - 1)
                assert np.all(loads >= 0) and np.all(loads < geo["units"])
                if us.size == 0:
                    continue
                # weight: unit u of the row, inside the row's bytes
                if qk == 32:
                    nb = np.minimum(LB, blocks - us * LB)
                    assert np.all(nb >= 1)
                    last = us * ubytes + nb * (ubytes // LB)
                else:
                    last = us * ubytes + ubytes
                assert np.all(last <= row_bytes)
                # MFMA operand reads: element k (8 halves) of activation row j
                for g in range(4):
                    if qk == 256:
                        if fmt == "q6_k":
                            offs = [128 * (g >> 1) + 32 * (st >> 1) + 16 * (g & 1) + 8 * (st & 1) for st in range(8)]
                        else:
                            offs = [64 * g + 8 * s for s in range(8)]
                        ks = (us[:, None] * 256 + np.array(offs)[None, :]).ravel()
                        widths = 8
                    else:
                        nbm = np.minimum(LB, blocks - us * LB)
                        ks_l = []
                        for bi in range(LB):
                            sel = us[nbm > bi]
                            kb = sel * 128 + 32 * bi
                            if fmt == "q8_0":
                                ks_l.append(kb + 8 * g)
                            else:  # 4 at kb + 4g, 4 at kb + 16 + 4g
                                ks_l += [kb + 4 * g, kb + 16 + 4 * g]
                        ks = np.concatenate(ks_l) if ks_l else np.zeros(0, np.int64)
                        widths = 8 if fmt == "q8_0" else 4
                    rel = ks - c0
                    assert np.all(rel >= 0) and np.all(rel + widths <= ln), "read outside the staged chunk"
                    for j in range(16):
                        row = j if j < mt else 0
                        idx = row * stride + rel
                        assert np.all(idx + widths <= mrows * stride)
                        assert np.all(staged[(idx[:, None] + np.arange(widths)).ravel()]), "read of unstaged LDS"
    return chunks


# The benchmark run that faulted: config 5's Qwen2.5-7B projections at
# m = 8 / 16 (then served by this kernel) and config 2's legacy shapes.
FAULT_RUN = [(fmt, m, n, k) for m in (8, 16)
             for fmt, n, k in (("q4_k", 3584, 3584), ("q4_k", 512, 3584), ("q6_k", 512, 3584),
                               ("q4_k", 18944, 3584), ("q6_k", 3584, 18944))]


@pytest.mark.parametrize("fmt,M,N,K", FAULT_RUN)
def test_gemv_geometry_fault_run_shapes(fmt, M, N, K):
    chunks = check_gemv(fmt, M, N, K, xt=0)
    assert chunks >= 2 if K > 3000 else True


@pytest.mark.parametrize("fmt", sorted(UNIT))
@pytest.mark.parametrize("M", [2, 5, 8, 16, 17, 40])
@pytest.mark.parametrize("K", [1536, 3584, 4096, 7168, 14336, 18944])
@pytest.mark.parametrize("xt", [0, 1])
def test_gemv_geometry_sweep(fmt, M, K, xt):
    if K % UNIT[fmt][2]:
        pytest.skip("k not a block multiple")
    check_gemv(fmt, M, 35, K, xt)


def test_gemv_geometry_reaches_many_chunks():
    # fp32 x at m = 16 stages 768 values per chunk: K = 18944 takes 25 chunks
    assert check_gemv("q4_k", 16, 33, 18944, 1) == 25
    assert check_gemv("q8_0", 16, 33, 14336, 0) == 9


def splitk_host(units, M, N, cus, mt=8, nt=1, nw=4, fmt="q4_k"):
    """launch_gemm2's slice count and scratch sizes (cq_host.cpp)."""
    slots = cus * (2 if mt == 8 and nw == 4 else 1)
    mblk = -(-M // (16 * mt))
    gx = -(-N // (16 * nw * nt))
    splits = 1
    if mt == 4:  # fewer than 1.5 workgroups per compute unit
        while 2 * gx * mblk * splits < 3 * cus and units // (splits * 2) >= 3:
            splits *= 2
    else:
        while gx * mblk * splits * 2 <= slots and units // (splits * 2) >= 3:
            splits *= 2
    splits = min(splits, units)
    usplit = -(-units // splits)
    splits = -(-units // usplit)
    sums = M * units * 32 if fmt != "q6_k" else 0
    part = splits * M * N * 4 if splits > 1 else 0
    return splits, usplit, sums, part


def test_gemm2_short_prefill_splits():
    # MT = 4 slice counts of the measured shapes (m = 17)
    assert splitk_host(16, 17, 14336, 256, mt=4)[0] == 2
    assert splitk_host(14, 17, 18944, 256, mt=4)[0] == 2
    assert splitk_host(56, 17, 4096, 256, mt=4)[0] == 8
    assert splitk_host(14, 17, 3584, 256, mt=4)[0] == 4


@pytest.mark.parametrize("N,K,M", [(512, 3584, 512), (512, 7168, 64), (3584, 18944, 512), (200, 2560, 130),
                                   (18944, 3584, 40),
                                   (1024, 4096, 17), (128, 65536, 2048)])
@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_gemm2_scratch_offsets(N, K, M, fmt):
    units = K // 256
    splits, usplit, sums, part = splitk_host(units, M, N, 256, mt=4 if M <= 64 else 8, fmt=fmt)
    # gemm2_body: slice z covers superblocks [z * usplit, min(+usplit, units))
    covered = []
    for z in range(splits):
        ub = z * usplit
        nu = min(usplit, units - ub)
        assert nu >= 1
        covered += list(range(ub, ub + nu))
        if sums:  # xs[(row * units + ub + u) * 16 + 8 * (lane & 1)], 8 halves
            hi = ((M - 1) * units + ub + nu - 1) * 16 + 8 + 8
            assert hi * 2 <= sums
        if part:  # part[(z * M + m) * N + n], fp32
            assert ((z * M + M - 1) * N + N - 1 + 1) * 4 <= part
    assert covered == list(range(units))
    if part:  # reduce: part[z * mn + i]
        assert ((splits - 1) * M * N + M * N) * 4 == part


SB_BYTES = {"q4_k": 144, "q5_k": 176, "q6_k": 210}


def gemm2_tile_host(fmt, M, N, K, cus=256):
    """launch_gemm2's tile choice (cq_host.cpp): (mt, nt, nw)."""
    units = K // 256
    wide = False
    if fmt == "q6_k" and M >= 256:
        t16 = -(-N // 128) * -(-M // 256)
        sp = 1
        while t16 * sp * 2 <= cus and units // (sp * 2) >= 3:
            sp *= 2
        wgs = t16 * sp
        rounds = -(-wgs // cus)
        wide = wgs * 5 >= rounds * cus * 4
    mt = 16 if wide else 4 if M <= 64 or (fmt == "q4_k" and M <= 128 and -(-N // 64) * -(-M // 64) >= cus) else 8
    nw = 8 if mt == 16 else 4
    slots = cus * {4: 4, 8: 2, 16: 1}[mt]
    if mt == 4:
        return mt, 1, nw
    mblk = -(-M // (16 * mt))
    fill = -(-N // (16 * nw)) * mblk * 2
    if wide:
        nt = 1
    elif fmt == "q6_k":
        nt = 2 if fill * 4 >= slots * 3 else 1
    else:
        nt = 2 if fill >= slots else 1
    return mt, nt, nw


@pytest.mark.parametrize("N,K,M,wide", [(4096, 14336, 512, True), (4096, 14336, 2048, True),
                                        (3584, 18944, 512, True), (14336, 4096, 256, True),
                                        (512, 3584, 512, False), (3584, 3584, 256, False),
                                        (18944, 3584, 512, False), (4096, 14336, 128, False)])
def test_gemm2_q6k_tile_choice(N, K, M, wide):
    # the Q6_K shapes measured for the MT = 16 rule (cq_host.cpp)
    mt, nt, nw = gemm2_tile_host("q6_k", M, N, K)
    assert (mt == 16) == wide
    if wide:
        assert (nt, nw) == (1, 8)


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
@pytest.mark.parametrize("M,mt", [(17, 4), (64, 4), (65, 8), (128, 8), (129, 8)])
def test_gemm2_short_prefill_tile(fmt, M, mt):
    # MT = 4 (one weight tile per wave) up to 64 activation rows, for Q4_K
    # weights that fill the compute units up to 128 (cq_host.cpp)
    if fmt == "q4_k" and 64 < M <= 128:
        mt = 4
    assert gemm2_tile_host(fmt, M, 4096, 14336)[0] == (4 if M <= 64 else 8)
    got_mt, nt, nw = gemm2_tile_host(fmt, M, 14336, 4096)
    assert (got_mt, nw) == (mt, 4)
    if mt == 4:
        assert nt == 1


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
@pytest.mark.parametrize("mt,nt,nw", [(4, 1, 4), (8, 1, 4), (8, 2, 4), (16, 1, 8), (16, 2, 8)])
@pytest.mark.parametrize("N,K", [(4096, 14336), (128256, 4096), (200, 2560), (3584, 65536)])
def test_gemm2_dma_cover_and_buffer_offsets(fmt, mt, nt, nw, N, K):
    # gemm2_body: activation DMA instruction i = wave + NW ii moves staged
    # rows 4i .. 4i + 3; the sums DMA instruction i < MT/2 moves rows
    # 32i .. 32i + 31; together they cover the workgroup's 16 MT rows once
    rows = sorted(4 * (wave + nw * ii) + r for wave in range(nw) for ii in range(4 * mt // nw) for r in range(4))
    assert rows == list(range(16 * mt))
    srows = sorted(32 * (wave + nw * ii) + r for wave in range(nw) for ii in range((mt // 2 + nw - 1) // nw)
                   if wave + nw * ii < mt // 2 for r in range(32))
    assert srows == list(range(16 * mt))
    # weight buffer loads: base = the workgroup's first row and slice; the
    # largest voffset + immediate + soffset stays under the 2^31 records
    units = K // 256
    row_bytes = units * SB_BYTES[fmt]
    rows_wg = nw * 16 * nt
    lane_max = {"q4_k": 32 + 16 + 16 + 64, "q5_k": 32 + 16 + 48 + 64, "q6_k": 208}[fmt]
    top = (rows_wg - 1) * row_bytes + lane_max + 16 + (units - 1) * SB_BYTES[fmt]
    assert top < 2 ** 31
