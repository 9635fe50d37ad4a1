"""Seeded synthetic inputs for the benchmark configurations.

Host generation uses numpy's Philox bit generator; one host buffer is fed to
both the GPU library and the CPU checker in the same run, so the two sides
always see identical bytes.  The 20M x 768 configuration is generated on the
device instead (vs_gen_normal, add_device_normal below); its rows are
checked against a host restatement of that generator on rows read back.

Normalisation follows L2NormTransform (l2_norm_transform.dart:23-46): fp64
sum of squares, inv = 1/sqrt, o = v * inv rounded to fp32 (zero rows stay
zero).  bf16 values are carried as uint16 bit patterns (round to nearest even).
"""
from __future__ import annotations

import numpy as np


def rng(seed: int, stream: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=seed, counter=[0, 0, 0, stream]))


def l2_normalize(x: np.ndarray) -> np.ndarray:
    """L2NormTransform.apply: the fp64 sum of squares in dimension order
    (an accumulating sum, not a pairwise one), norm = sqrt, inv = 1 / norm,
    fp32(v * inv); zero rows stay zero."""
    from .wrappers import L2NormTransform

    return L2NormTransform(x.shape[1]).apply(np.asarray(x, np.float32))


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def normal_unit(n: int, d: int, seed: int, stream: int) -> np.ndarray:
    """N(0,1) rows, L2-normalised (configs 1, 3, 5)."""
    return l2_normalize(rng(seed, stream).standard_normal((n, d), dtype=np.float32))


def int_grid(n: int, d: int, seed: int, stream: int) -> np.ndarray:
    """Uniform integers 0..255 stored as fp32 (config 2)."""
    return rng(seed, stream).integers(0, 256, size=(n, d), dtype=np.int32).astype(np.float32)


def gaussian_mixture(n: int, d: int, ncomp: int, sigma: float, seed: int):
    """Config 4: centres N(0,1); point = centre[uniform component] + N(0, sigma^2)."""
    g = rng(seed, 0)
    centres = g.standard_normal((ncomp, d), dtype=np.float32)
    comp = rng(seed, 1).integers(0, ncomp, size=n)
    noise = rng(seed, 2).standard_normal((n, d), dtype=np.float32) * np.float32(sigma)
    return (centres[comp] + noise).astype(np.float32), comp


def seeded_subset(n: int, k: int, seed: int) -> np.ndarray:
    """k distinct indices of [0, n) (partial Fisher-Yates via Generator.choice)."""
    return rng(seed, 3).choice(n, size=k, replace=False)


def dedup_set(n: int, d: int, dup_frac: float, noise: float, seed: int) -> np.ndarray:
    """Config 5: (1 - dup_frac) n unit base vectors, dup_frac n copies of random
    bases + N(0, noise^2) renormalised, rows shuffled by a seeded permutation."""
    ndup = int(round(n * dup_frac))
    nbase = n - ndup
    base = normal_unit(nbase, d, seed, 0)
    src = rng(seed, 1).integers(0, nbase, size=ndup)
    cop = base[src] + rng(seed, 2).standard_normal((ndup, d), dtype=np.float32) * np.float32(noise)
    allv = np.concatenate([base, l2_normalize(cop)], axis=0)
    perm = rng(seed, 3).permutation(n)
    return np.ascontiguousarray(allv[perm])


def dedup_planted_pairs(n: int, dup_frac: float, seed: int):
    """Every pair (i, j), i < j, of rows of dedup_set(n, ..., dup_frac, ...,
    seed) that hold the same base vector or copies of it (the generator's
    planted near-duplicates), as two int64 arrays sorted by (i, j)."""
    ndup = int(round(n * dup_frac))
    nbase = n - ndup
    src = rng(seed, 1).integers(0, nbase, size=ndup)
    perm = rng(seed, 3).permutation(n)
    row = np.empty(n, np.int64)
    row[perm] = np.arange(n)  # row of generated vector v: row[v]
    order = np.argsort(src, kind="stable")
    pi, pj = [], []
    start = 0
    while start < ndup:
        b = src[order[start]]
        end = start
        while end < ndup and src[order[end]] == b:
            end += 1
        members = np.sort(np.concatenate(([row[b]], row[nbase + order[start:end]])))
        for a in range(len(members)):
            for c in range(a + 1, len(members)):
                pi.append(members[a])
                pj.append(members[c])
        start = end
    pi, pj = np.asarray(pi, np.int64), np.asarray(pj, np.int64)
    o = np.lexsort((pj, pi))
    return pi[o], pj[o]


DEVICE_STREAM_BASE = 1 << 32


def add_device_normal(idx, n: int, d: int, seed: int, chunk: int = 1 << 20) -> None:
    """Fill a bf16 index with n L2-normalised N(0,1) rows made on the device
    (config 3's database): rows [r, r + chunk) come from vs_gen_normal with
    stream DEVICE_STREAM_BASE + r and row counters 0 .. chunk - 1."""
    from . import _native as NN

    idx.reserve(n)
    buf = NN.DeviceBuffer(min(chunk, n) * d * 2)
    try:
        for r in range(0, n, chunk):
            m = min(chunk, n - r)
            NN.check(NN.load().vs_gen_normal(0, buf.ptr, NN.VS_DTYPE_BF16, m, d, seed,
                                             DEVICE_STREAM_BASE + r, 1))
            idx.add_device(buf, m, NN.VS_DTYPE_BF16)
    finally:
        buf.free()
