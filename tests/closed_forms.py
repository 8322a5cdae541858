"""Float64 closed forms of the C3 functions (the BASELINE configuration's anvil.function calls), and
their inputs: ~N(0,1) float32 from a seeded generator, as BASELINE.json states them."""
import numpy as np


def softmax_case(seed=2):
    x = np.random.default_rng(seed).standard_normal((8192, 4096)).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    return [x], e / e.sum(axis=1, keepdims=True)


def layernorm_case(seed=2):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((8192, 1024)).astype(np.float32)
    g = rng.standard_normal(1024).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=1, keepdims=True)
    return [x, g, b], (x64 - mu) / np.sqrt(var + 1e-5) * g + b


LINEAR_ROWS = 128 * np.arange(64) + (37 * np.arange(64)) % 128      # one row of each 128-row tile


def linear_case(seed=2):
    """y = x·Wᵀ + b at [8192, 4096] x [4096, 4096]; the closed form for LINEAR_ROWS only."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((8192, 4096)).astype(np.float32)
    w = rng.standard_normal((4096, 4096)).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    return [x, w, b], x[LINEAR_ROWS].astype(np.float64) @ w.astype(np.float64).T + b


def attention_case(seed=2):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((4, 2048, 128)).astype(np.float32) for _ in range(3))
    s = np.matmul(q.astype(np.float64), k.astype(np.float64).transpose(0, 2, 1)) / np.sqrt(128.0)
    p = np.exp(s - s.max(axis=2, keepdims=True))
    return [q, k, v], np.matmul(p / p.sum(axis=2, keepdims=True), v.astype(np.float64))
