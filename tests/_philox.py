"""Host restatement of the library's device generator (vs_gen_normal), for
checking rows it wrote: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11),
fp64 Box-Muller rounded to fp32, and the L2NormTransform normalisation
(lib/core/vector_store/l2_norm_transform.dart:23-46: fp64 sum of squares in
dimension order, inv = 1 / sqrt, fp32(v * inv)), then bf16 round to nearest
even.  Test infrastructure only.
"""
import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """ctr: uint32 array (..., 4); key: (k0, k1).  Returns uint32 (..., 4)."""
    c = [np.asarray(ctr[..., i], np.uint64) for i in range(4)]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
        k0 = (k0 + W0) & 0xFFFFFFFF
        k1 = (k1 + W1) & 0xFFFFFFFF
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def _box_muller(a, b):
    u1 = ((a >> np.uint32(8)).astype(np.float64) + 1.0) * (1.0 / 16777216.0)
    u2 = (b >> np.uint32(8)).astype(np.float64) * (1.0 / 16777216.0)
    r = np.sqrt(-2.0 * np.log(u1))
    t = 6.283185307179586 * u2
    return (r * np.cos(t)).astype(np.float32), (r * np.sin(t)).astype(np.float32)


def raw_rows(rows, d, seed, stream):
    """N(0,1) fp32 values of the given rows, before normalisation."""
    rows = np.asarray(rows, np.uint64)
    groups = (d + 3) // 4
    g = rows[:, None] * np.uint64(groups) + np.arange(groups, dtype=np.uint64)[None, :]
    ctr = np.stack([g & MASK, g >> np.uint64(32),
                    np.full_like(g, stream & 0xFFFFFFFF), np.full_like(g, stream >> 32)], axis=-1)
    r = philox4x32_10(ctr.astype(np.uint32), (seed & 0xFFFFFFFF, seed >> 32))
    z0, z1 = _box_muller(r[..., 0], r[..., 1])
    z2, z3 = _box_muller(r[..., 2], r[..., 3])
    z = np.stack([z0, z1, z2, z3], axis=-1).reshape(len(rows), groups * 4)
    return z[:, :d]


def normalized_rows(rows, d, seed, stream):
    """fp32 rows as vs_gen_normal(normalize=1) computes them before bf16 rounding."""
    z = raw_rows(rows, d, seed, stream)
    out = np.empty_like(z)
    for i in range(z.shape[0]):
        s = 0.0
        for v in z[i].astype(np.float64):  # dimension order, as the reference sums
            s = s + v * v
        norm = np.sqrt(s)
        inv = 1.0 / norm if norm > 0 else 0.0
        out[i] = (z[i].astype(np.float64) * inv).astype(np.float32)
    return out
