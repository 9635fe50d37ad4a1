"""Host restatement of the LDS-DMA GEMM kernel's address arithmetic
(gemm_dma_kernel / issue() / dma16 / dma16_lane in
dart-pytorch_amd/csrc/vs_gemm.hip) for the case that faulted on its first
GPU run: shape (query planes 1, row waves 2, query waves 4, 32-row blocks 4,
32-query blocks 2, 4 stages), 9,000 bf16 rows of d = 200 (ld = 256),
300 queries, L2, k = 10.  The kernel stays switched off; this test records
what reading the code shows, on the CPU:

- every global byte the DMA loads read lies inside its buffer (rows below
  capacity + kRowSlack, query plane rows below the padded query count,
  norms and thresholds inside theirs);
- every LDS byte it intends to write lies inside the dynamic allocation and
  below the list counters that follow the stages;
- but stage 3's targets run past 2^17 bytes (and stages 1-3 past 2^16): if
  the hardware took fewer bits of M0 for the LDS address, or a lane index
  across the workgroup instead of the wave, the writes would land elsewhere;
  under the second reading some land on the list counters, whose corrupted
  values would index the global candidate lists out of range.  Neither
  reading is confirmed, so no cause is shown.
"""
K_ROW_SLACK = 512


def dma_case():
    pb, wr, wq, rb, qb, ns = 1, 2, 4, 4, 2, 4
    nw, br, bq = wr * wq, wr * 32 * rb, wq * 32 * qb
    a_ins, b_ins = br * 64 // 1024, pb * bq * 64 // 1024
    a_pw, b_pw = a_ins // nw, b_ins // nw
    a_bytes, b_bytes = br * 64, pb * bq * 64
    n_off = a_bytes + b_bytes
    g_off = n_off + br * 4
    stage = g_off + bq * 4
    kk_final = 16  # next_pow2(k + max(4, k // 4)) for k = 10
    cap = 1 << (kk_final + 32 * rb + 16 - 1).bit_length()
    lds_total = ns * stage + wr * bq * 8 + nw * cap * 8
    counters = ns * stage
    # index: 9,000 rows (capacity rounded to 256), ld 256, queries padded
    n, d, ld, nq = 9000, 200, 256, 300
    cap_rows = -(-max(n, 1024) // 256) * 256
    nq_pad = -(-nq // 256) * 256 + 256
    return dict(pb=pb, wr=wr, wq=wq, rb=rb, qb=qb, ns=ns, nw=nw, br=br, bq=bq, a_pw=a_pw,
                b_pw=b_pw, a_bytes=a_bytes, n_off=n_off, g_off=g_off, stage=stage,
                lds_total=lds_total, counters=counters, n=n, ld=ld, nq=nq, cap_rows=cap_rows,
                nq_pad=nq_pad)


def swz(r):
    return ((r >> 1) ^ (r >> 2)) & 3


def test_dma_addresses_in_range():
    c = dma_case()
    row_bytes = c["ld"] * 2
    # plan: 2 query blocks, splits of 1,280 rows (the last one 40 rows)
    nqblk = -(-c["nq"] // c["bq"])
    rps, nsplit = 1280, -(-c["n"] // 1280)
    lds_hi = 0
    for split in range(nsplit):
        r0, r1 = split * rps, min(c["n"], split * rps + rps)
        ntiles = -(-(r1 - r0) // c["br"])
        for qblk in range(nqblk):
            q0 = qblk * c["bq"]
            for tile in range(ntiles):
                t = r0 + tile * c["br"]
                for kc in range(c["ld"] // 32):
                    for st in range(c["ns"]):
                        sb = st * c["stage"]
                        for wave in range(c["nw"]):
                            for lane in range(64):
                                for j in range(c["a_pw"]):
                                    r = 16 * (wave * c["a_pw"] + j) + (lane >> 2)
                                    g = (t + r) * row_bytes + kc * 64 + 16 * ((lane & 3) ^ swz(r))
                                    assert 0 <= g and g + 16 <= (c["cap_rows"] + K_ROW_SLACK) * row_bytes
                                    lo = sb + (wave * c["a_pw"] + j) * 1024 + 16 * lane
                                    lds_hi = max(lds_hi, lo + 16)
                                for j in range(c["b_pw"]):
                                    brow = 16 * (wave * c["b_pw"] + j) + (lane >> 2)
                                    p, q = brow // c["bq"], brow % c["bq"]
                                    plane_row = 2 * (q0 + q) + p
                                    assert plane_row < 2 * c["nq_pad"]
                                    lo = sb + c["a_bytes"] + (wave * c["b_pw"] + j) * 1024 + 16 * lane
                                    lds_hi = max(lds_hi, lo + 16)
                            if kc == 0:
                                # norms (wave 0, 256 floats) and thresholds (last wave, 256 words)
                                assert t + 256 <= c["cap_rows"] + K_ROW_SLACK
                                assert q0 + c["bq"] <= c["nq_pad"]
                                lds_hi = max(lds_hi, sb + c["n_off"] + 1024,
                                             sb + c["g_off"] + 1024)
    assert lds_hi <= c["counters"] <= c["lds_total"] <= 160 * 1024
    # the intended targets run past 2^16 and 2^17 bytes of LDS
    assert lds_hi > 1 << 17


def test_workgroup_lane_reading_reaches_the_counters():
    """Under the (unconfirmed) reading LDS address = M0 + 16 x (thread index
    in the workgroup), wave 6's second B load of stage 3 lands on the list
    counters that follow the stages."""
    c = dma_case()
    sb = 3 * c["stage"]
    wave, j = 6, 1
    base = sb + c["a_bytes"] + (wave * c["b_pw"] + j) * 1024
    lo, hi = base + 16 * (64 * wave), base + 16 * (64 * wave + 63) + 16
    assert lo < c["counters"] + c["wr"] * c["bq"] * 4 and hi > c["counters"]
