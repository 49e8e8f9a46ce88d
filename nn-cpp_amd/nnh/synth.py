"""Synthetic inputs with the reference's own seeded streams.

nn-cpp's bench and tests fill operands in row-major order from std::mt19937(seed) through
std::uniform_real_distribution<float>(lo, hi) (apps/bench/runner.cpp:80-86, tests/test_kernels.cpp:75-83).
libstdc++ maps one 32-bit draw u to float(u) / 2^32 (generate_canonical<float, 24>, clamped below 1),
then to c * (hi - lo) + lo in float arithmetic. mt19937_uniform reproduces that stream bit for bit with
numpy's MT19937 under the same init_genrand seeding, so the GPU and the CPU reference see identical bytes.
"""
import numpy as np


def mt19937_raw(seed, count):
    bg = np.random.MT19937(0)
    bg._legacy_seeding(int(seed))
    return bg.random_raw(int(count)).astype(np.uint32)


def uniform_from_raw(raw, lo, hi):
    """uniform_real_distribution<float>(lo, hi) applied to 32-bit draws raw (libstdc++'s mapping)."""
    c = raw.astype(np.float32) / np.float32(4294967296.0)
    c = np.where(c >= np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0.0)), c).astype(np.float32)
    span = np.float32(np.float32(hi) - np.float32(lo))
    return (c * span + np.float32(lo)).astype(np.float32)


def mt19937_uniform(seed, count, lo=-1.0, hi=1.0):
    return uniform_from_raw(mt19937_raw(seed, count), lo, hi)


def reseeded_parameters(seed, shapes, ones=()):
    """apps/bench/workloads.cpp:28-43 reseed_parameters: one std::mt19937(seed) stream over the parameters in order;
    a parameter of rank < 2 becomes zeros (no draws), or stays all ones when its index is in `ones` (keep_ones_rank1
    for parameters initialised to one, as LayerNorm's gamma is); any other U(+-1/sqrt(size / shape[0])) in row-major
    order."""
    sizes = [int(np.prod(s)) for s in shapes]
    raw = mt19937_raw(seed, sum(n for s, n in zip(shapes, sizes) if len(s) >= 2))
    out, off = [], 0
    for i, (s, n) in enumerate(zip(shapes, sizes)):
        if len(s) < 2:
            out.append(np.ones(s, np.float32) if i in ones else np.zeros(s, np.float32))
            continue
        bound = np.float32(1.0) / np.sqrt(np.float32(n // s[0]))
        out.append(np.ascontiguousarray(uniform_from_raw(raw[off:off + n], -bound, bound).reshape(s)))
        off += n
    return out


def uniform_operands(seed, shapes, lo=-1.0, hi=1.0):
    """Consecutive draws of one stream, one array per shape (run_matmul fills A, then B)."""
    sizes = [int(np.prod(s, dtype=np.int64)) for s in shapes]
    flat = mt19937_uniform(seed, sum(sizes), lo, hi)
    out, off = [], 0
    for s, n in zip(shapes, sizes):
        out.append(flat[off:off + n].reshape(s))
        off += n
    return out


def normal(seed, shape):
    """N(0, 1) float32 values (numpy's PCG64 stream; both sides receive the same buffer)."""
    return np.random.default_rng(seed).standard_normal(size=shape, dtype=np.float32)


def uniform_ids(seed, count, bits):
    """std::uniform_int_distribution<int>(0, 2^bits - 1) over std::mt19937(seed), as libstdc++ 11 draws it
    (multiply-shift: (r * 2^bits) >> 32, which for a power-of-two range keeps the top `bits` bits of each output and
    never rejects), as floats: the token ids of apps/bench/workloads.cpp:85-87."""
    return (mt19937_raw(seed, count) >> np.uint32(32 - bits)).astype(np.float32)
