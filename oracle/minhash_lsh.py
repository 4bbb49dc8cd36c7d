"""Restatement of the LSH library the reference's TCA reorder calls -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__).

The reference imports MinHash and MinHashLSH from the third-party package datasketch
(spmm/tr_csr_fp16/tr_tca_reorder.py:15, used at :84-90, :121-123, :226-249); the package is not
vendored in the reference, which pins no version, and it is not installed here.  Its published
algorithm (the MinHash / MinHashLSH defaults of its 1.x releases), restated:

  * MinHash(num_perm=128, seed=1, hashfunc=sha1_hash32): hash values start at 2^32 - 1; the
    permutations are num_perm pairs (a, b) drawn in that order by numpy's legacy
    RandomState(seed): a = randint(1, 2^61 - 1), b = randint(0, 2^61 - 1), uint64;
    update(x): hv = the first 4 bytes of SHA-1(x) read little-endian; per permutation
    ((a * hv + b) mod 2^64) mod (2^61 - 1), low 32 bits; values = elementwise minimum.
    The reference updates with str(column).encode('utf-8').
  * MinHashLSH(threshold, num_perm, weights=(0.5, 0.5)): (b, r) minimising
    0.5 * integral_0^t (1 - (1 - s^r)^b) ds + 0.5 * integral_t^1 (1 - s^r)^b ds over b in
    [1, num_perm], r in [1, num_perm // b] (first minimum in that loop order, scipy quad); band i
    is values[i r : (i + 1) r]; a query returns every inserted key sharing at least one band.

What pins it here: numpy's RandomState and hashlib are the real implementations of the two
primitives; the rest is the formulas above.  The candidate sets of the reference follow from the
signatures alone; its queue order for equal similarities does not (tr_tca_reorder.py:116-130
iterates a Python set of strings, whose order changes with the per-process string hash).
"""
from __future__ import annotations

import hashlib
import struct

import numpy as np

MERSENNE = np.uint64((1 << 61) - 1)
MAX_HASH = np.uint64((1 << 32) - 1)


def sha1_hash32(data: bytes) -> int:
    return struct.unpack("<I", hashlib.sha1(data).digest()[:4])[0]


def permutations(num_perm: int = 128, seed: int = 1):
    gen = np.random.RandomState(seed)
    pairs = [(gen.randint(1, MERSENNE, dtype=np.uint64), gen.randint(0, MERSENNE, dtype=np.uint64))
             for _ in range(num_perm)]
    a = np.array([p[0] for p in pairs], dtype=np.uint64)
    b = np.array([p[1] for p in pairs], dtype=np.uint64)
    return a, b


def minhash(elements, num_perm: int = 128, seed: int = 1, perms=None) -> np.ndarray:
    a, b = perms if perms is not None else permutations(num_perm, seed)
    values = np.full(num_perm, MAX_HASH, dtype=np.uint64)
    with np.errstate(over="ignore"):
        for e in elements:
            hv = np.uint64(sha1_hash32(str(int(e)).encode("utf-8")))
            phv = np.bitwise_and((a * hv + b) % MERSENNE, MAX_HASH)
            values = np.minimum(phv, values)
    return values


def optimal_param(threshold: float, num_perm: int, fp_weight: float = 0.5, fn_weight: float = 0.5):
    from scipy.integrate import quad

    def fp(b, r):
        return quad(lambda s: 1 - (1 - s ** float(r)) ** float(b), 0.0, threshold)[0]

    def fn(b, r):
        return quad(lambda s: 1 - (1 - (1 - s ** float(r)) ** float(b)), threshold, 1.0)[0]

    best, opt = float("inf"), (0, 0)
    for b in range(1, num_perm + 1):
        for r in range(1, num_perm // b + 1):
            err = fp(b, r) * fp_weight + fn(b, r) * fn_weight
            if err < best:
                best, opt = err, (b, r)
    return opt


def candidate_pairs(sets, threshold: float = 0.2, num_perm: int = 128, seed: int = 1, bands=None) -> list:
    """Pairs (i, j), i < j, of non-empty sets that the LSH pairs up (every set inserted, every
    non-empty set queried, as the reference does at :84-90 and :119-130)."""
    b, r = bands if bands is not None else optimal_param(threshold, num_perm)
    perms = permutations(num_perm, seed)
    sigs = [minhash(s, num_perm, seed, perms) for s in sets]
    tables = [dict() for _ in range(b)]
    for i, v in enumerate(sigs):
        for t in range(b):
            tables[t].setdefault(v[t * r:(t + 1) * r].tobytes(), []).append(i)
    pairs = set()
    for i, v in enumerate(sigs):
        if not sets[i]:
            continue
        for t in range(b):
            for j in tables[t][v[t * r:(t + 1) * r].tobytes()]:
                if j != i and sets[j]:
                    pairs.add((min(i, j), max(i, j)))
    return sorted(pairs)
