"""The training attention's kernels (hip_rt/anvil_attn_train.h) against float64, at shapes the C4
fixtures do not reach.

tests/attn_train_check.hip (built by __graft_entry__.build()) launches the forward, dQ and dK/dV
kernels on device buffers in the generated code's layout. Here the results are compared with a
float64 NumPy evaluation of the definitions: S = alpha·Q Kᵀ with keys past the query masked, P its
row softmax, O = P V; dP = dO Vᵀ, dS = P ⊙ (dP − rowsum(dP ⊙ P)), dQ = alpha·dS K, dK = alpha·dSᵀ Q,
dV = Pᵀ dO, with the backward as two launches and as one. The shapes cover one tile per workgroup (T = 64),
pairs of tiles with an odd middle one
(T = 96, 160), staging in rounds of four and in one round of eight, heads of 32 and 64, and a batch ×
heads count that is not a multiple of 8 (the workgroups then go to the XCDs in plain order). The C4
programs of tests/test_hip_gpu.py hold the same kernels to the reference interpreter's vectors.
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "anvil-lang_amd", "anvil", "_libs",
                   "attn_train_check.so")
LOG2E = 1.4426950408889634


def _lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB)
    lib.attn_train_check.restype = ctypes.c_int
    lib.attn_train_check.argtypes = [ctypes.c_int] * 6 + [ctypes.c_float] + [ctypes.c_void_p] * 7
    lib.attn_train_check_error.restype = ctypes.c_char_p
    return lib


def _shapes(lib):
    buf = (ctypes.c_int * 96)()
    n = lib.attn_train_check_shapes(buf, 96)
    return [tuple(buf[3 * i:3 * i + 3]) for i in range(n)]


def _reference(q, k, v, do, alpha):
    """Per head [T, D] float64 arrays: O, m, l, dQ, dK, dV."""
    T = q.shape[0]
    s = alpha * q @ k.T
    s[np.triu_indices(T, 1)] = -np.inf
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=1, keepdims=True)
    p = e / l
    o = p @ v
    dp = do @ v.T
    ds = p * (dp - (dp * p).sum(axis=1, keepdims=True))
    return o, m[:, 0], l[:, 0], alpha * ds @ k, alpha * ds.T @ q, p.T @ do


def test_the_library_instantiates_the_plan_choices():
    """Every (D, T) that a C4-like program can bring runs through one of these instantiations with
    the tile grouping the plan picks for it (one tile per workgroup where a head has two or fewer)."""
    shapes = _shapes(_lib())
    assert shapes and all(d in (32, 64) and (ti == 1) == (nt <= 2) for d, nt, ti in shapes)


@pytest.mark.parametrize("combined", [0, 1])
@pytest.mark.parametrize("B,H", [(2, 3)])
def test_kernels_match_float64(B, H, combined):
    from anvil.hip_function import DeviceArray          # the HIP runtime the libraries link
    lib = _lib()
    rng = np.random.default_rng(5)
    for D, NT, TI in _shapes(lib):
        T = 32 * NT
        alpha = 1.0 / np.sqrt(D)
        qkv = rng.standard_normal((B, T, 3, H, D)).astype(np.float32)
        do = rng.standard_normal((B, T, H, D)).astype(np.float32)
        nan = lambda shape: DeviceArray.from_host(np.full(shape, np.nan, np.float32))
        ins = {"qkv": DeviceArray.from_host(qkv), "do": DeviceArray.from_host(do)}
        out = {"o": nan((B, T, H, D)), "m": nan((B, H, T)), "l": nan((B, H, T)), "drow": nan((B, H, T)),
               "dqkv": nan((B, T, 3, H, D))}
        try:
            print(f"attention kernels D={D} T={T} TI={TI} B={B} H={H} backward in one launch: {combined}", flush=True)
            rc = lib.attn_train_check(D, NT, TI, combined, B, H, alpha, ins["qkv"].data_ptr(), out["o"].data_ptr(),
                                      out["m"].data_ptr(), out["l"].data_ptr(), ins["do"].data_ptr(),
                                      out["drow"].data_ptr(), out["dqkv"].data_ptr())
            assert rc == 0, (D, NT, TI, rc, lib.attn_train_check_error().decode())
            got = {name: d.to_host().astype(np.float64) for name, d in out.items()}
        finally:
            for d in list(ins.values()) + list(out.values()):
                d.free()
        for n in range(B):
            for h in range(H):
                q, k, v = (qkv[n, :, i, h].astype(np.float64) for i in range(3))
                o, m, l, dq, dk, dv = _reference(q, k, v, do[n, :, h].astype(np.float64), alpha)
                where = f"D={D} T={T} TI={TI} combined={combined} n={n} h={h}"
                np.testing.assert_allclose(got["o"][n, :, h], o, rtol=0, atol=2e-6 * np.abs(o).max(), err_msg=where)
                # m is the row maximum in base 2 (scores scaled by log2 e)
                np.testing.assert_allclose(got["m"][n, h] / LOG2E, m, rtol=2e-6, atol=2e-6, err_msg=where)
                np.testing.assert_allclose(got["l"][n, h], l, rtol=5e-6, err_msg=where)
                for x, want, what in ((0, dq, "dQ"), (1, dk, "dK"), (2, dv, "dV")):
                    np.testing.assert_allclose(got["dqkv"][n, :, x, h], want, rtol=0, atol=4e-6 * np.abs(want).max(),
                                               err_msg=f"{what} {where}")
