"""nn-cpp's bench models as the training-step harnesses run them (apps/bench/workloads.cpp:28-137): parameter
shapes in parameter order, the reseeded parameters, the input, and a fixed gradient of the logits; and one call of a
harness's step entry (nnh_bench_workload_step in lib/libnnh_workloads.so on the GPU, nnref_time_workload_step on
the CPU), which both take (model, x, N, params, g, warmup, runs, fwd_ms, bwd_ms, logits, grads)."""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import synth


def transformer_tiny_shapes(vocab=64, dim=64, layers=2, mlp_ratio=4):
    """Transformer::named_parameters order (src/nn/transformer.cpp:51-58, 79-87): embed.weight; per block ln1 gamma
    beta, attn q k v o (weight, bias each), ln2 gamma beta, fc1 weight bias, fc2 weight bias; ln_f gamma beta, head
    weight bias. Returns (shapes, indices of the LayerNorm gammas, which start at one)."""
    shapes, ones = [(vocab, dim)], []
    for _ in range(layers):
        ones.append(len(shapes))
        shapes += [(dim,), (dim,)]
        shapes += [(dim, dim), (dim,)] * 4
        ones.append(len(shapes))
        shapes += [(dim,), (dim,), (mlp_ratio * dim, dim), (mlp_ratio * dim,), (dim, mlp_ratio * dim), (dim,)]
    ones.append(len(shapes))
    shapes += [(dim,), (dim,), (vocab, dim), (vocab,)]
    return shapes, tuple(ones)


@dataclass
class Workload:
    name: str
    model: int            # the harnesses' model index
    batch: int
    x_shape: tuple
    shapes: list
    out_shape: tuple      # the logits
    ones: tuple = ()      # rank-1 parameters that start at one
    ids: bool = False     # x holds token ids


_TF_SHAPES, _TF_ONES = transformer_tiny_shapes()

WORKLOADS = [
    Workload("mlp_wide", 0, 256, (256, 784), [(1024, 784), (1024,), (1024, 1024), (1024,), (10, 1024), (10,)],
             (256, 10)),
    Workload("cnn_mnist", 1, 32, (32, 1, 28, 28), [(8, 1, 3, 3), (8,), (16, 8, 3, 3), (16,), (128, 784), (128,),
                                                   (10, 128), (10,)], (32, 10)),
    Workload("transformer_tiny", 2, 16, (16, 64), _TF_SHAPES, (16 * 64, 64), _TF_ONES, ids=True),
]


def by_name(name):
    return next(w for w in WORKLOADS if w.name == name)


def inputs(w, seed=1):
    """make_workload's data for seed: parameters reseeded from std::mt19937(seed) (transformer_tiny keeping its
    gammas at one), x from std::mt19937(seed + 1) (U[0, 1) pixels, or ids in [0, 64)), and a N(0, 1) gradient of the
    logits from seed + 2."""
    params = synth.reseeded_parameters(seed, w.shapes, w.ones)
    n = int(np.prod(w.x_shape))
    x = (synth.uniform_ids(seed + 1, n, 6) if w.ids else synth.mt19937_uniform(seed + 1, n, 0.0, 1.0)).reshape(w.x_shape)
    g = synth.normal(seed + 2, w.out_shape)
    return params, x, g


def run_step(fn, w, params, x, g, warmup, runs, want_grads=False):
    """One call of a harness's step entry `fn`; returns (rc, fwd_ms, bwd_ms, logits, grads or None)."""
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    dp = lambda a: a.ctypes.data_as(C.POINTER(C.c_double))
    pp = (C.POINTER(C.c_float) * len(params))(*[fp(p) for p in params])
    fwd, bwd = np.empty(runs), np.empty(runs)
    logits = np.empty(w.out_shape, np.float32)
    grads = [np.full(s, np.nan, np.float32) for s in w.shapes] if want_grads else None
    gp = (C.POINTER(C.c_float) * len(params))(*[fp(a) for a in grads]) if want_grads else None
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(g, np.float32)
    rc = fn(w.model, fp(x), C.c_size_t(w.batch), pp, fp(g), warmup, runs, dp(fwd), dp(bwd), fp(logits), gp)
    return rc, fwd, bwd, logits, grads
