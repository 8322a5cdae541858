// Test library for tests/test_attn_train_gpu.py: the training attention's three kernels
// (anvil-lang_amd/anvil/backend/hip_rt/anvil_attn_train.h) launched on caller-provided device
// buffers, for shapes the C4 fixtures do not reach. Built by __graft_entry__.build().
//
// Layout (the generated code's, for Q, K, V held in one [B, T, 3, H, D] buffer): element (n, t, h, c)
// of Q at n·T·3HD + t·3HD + h·D + c, K at +HD, V at +2HD; O and dO [B, T, H, D]; m, l, Drow [B, H, T].
#include <hip/hip_runtime.h>
#include "../anvil-lang_amd/anvil/backend/hip_rt/anvil_mfma.h"
#include "../anvil-lang_amd/anvil/backend/hip_rt/anvil_attn_train.h"

template <int D, int NT, int TI>
__global__ void __launch_bounds__(256 * TI) at_fwd(anvil_attn_io a) { anvil_attn_fwd<D, NT, TI>(a); }
template <int D, int NT, int TI>
__global__ void __launch_bounds__(256 * TI) at_dq(anvil_attn_io a) { anvil_attn_bwd_q<D, NT, TI, false>(a); }
template <int D, int NT, int TI>
__global__ void __launch_bounds__(256 * TI) at_dkv(anvil_attn_io a) { anvil_attn_bwd_kv<D, NT, TI, false>(a); }

static hipError_t last_error = hipSuccess;

extern "C" const char *attn_train_check_error(void) { return hipGetErrorString(last_error); }

template <int D, int NT, int TI>
__global__ void __launch_bounds__(256 * TI) at_bwd(anvil_attn_io a) { anvil_attn_bwd<D, NT, TI, false>(a); }

// the backward as two launches (dQ writing Drow, then dK/dV) or, combined, as one launch of both
// kinds of workgroup
template <int D, int NT, int TI>
static int run(anvil_attn_io a, int BH, int combined) {
    const dim3 grid(anvil_at_groups(NT, TI) * BH), block(256 * TI);
    hipLaunchKernelGGL((at_fwd<D, NT, TI>), grid, block, 0, 0, a);
    if ((last_error = hipGetLastError()) != hipSuccess) return -3;
    if (combined) {
        a.drow = nullptr;
        hipLaunchKernelGGL((at_bwd<D, NT, TI>), dim3(2 * grid.x), block, 0, 0, a);
        if ((last_error = hipGetLastError()) != hipSuccess) return -4;
    } else {
        hipLaunchKernelGGL((at_dq<D, NT, TI>), grid, block, 0, 0, a);
        if ((last_error = hipGetLastError()) != hipSuccess) return -4;
        hipLaunchKernelGGL((at_dkv<D, NT, TI>), grid, block, 0, 0, a);
        if ((last_error = hipGetLastError()) != hipSuccess) return -5;
    }
    return (last_error = hipDeviceSynchronize()) == hipSuccess ? 0 : -2;
}

// The shapes this library instantiates: (D, NT, TI). Returns -1 for any other.
#define ANVIL_AT_SHAPES(X) X(64, 2, 1) X(64, 3, 2) X(64, 4, 2) X(64, 5, 2) X(64, 8, 2) X(32, 1, 1) X(32, 4, 2) X(32, 8, 2)

extern "C" int attn_train_check_shapes(int *out, int cap) {
    int n = 0;
#define ANVIL_AT_LIST(d, nt, ti) if (n + 3 <= cap) { out[n] = d; out[n + 1] = nt; out[n + 2] = ti; } n += 3;
    ANVIL_AT_SHAPES(ANVIL_AT_LIST)
#undef ANVIL_AT_LIST
    return n / 3;
}

// The forward, then the backward (combined or not): O, m (base 2), l, dQKV (and Drow when not
// combined) written.
extern "C" int attn_train_check(int D, int NT, int TI, int combined, int B, int H, float alpha, const float *qkv,
                                float *o, float *m, float *l, const float *dout, float *drow, float *dqkv) {
    const int T = 32 * NT, HD = H * D;
    anvil_attn_io a;
    a.q = qkv; a.k = qkv + HD; a.v = qkv + 2 * HD;
    a.qn = (long long)T * 3 * HD; a.qh = D; a.qs = 3 * HD;
    a.o = o; a.dout = dout; a.on = (long long)T * HD; a.oh = D; a.os = HD;
    a.m = m; a.l = l; a.drow = drow;
    a.dq = dqkv; a.dk = dqkv + HD; a.dv = dqkv + 2 * HD;
    a.H = H; a.BH = B * H; a.alpha = alpha;
#define ANVIL_AT_RUN(d, nt, ti) if (D == d && NT == nt && TI == ti) return run<d, nt, ti>(a, B * H, combined);
    ANVIL_AT_SHAPES(ANVIL_AT_RUN)
#undef ANVIL_AT_RUN
    return -1;
}
