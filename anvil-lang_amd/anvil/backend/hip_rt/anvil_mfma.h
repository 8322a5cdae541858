// anvil_mfma.h — fp32 matrix products on CDNA4 matrix cores (v_mfma_f32_32x32x2f32), for the
// contractions the HIP backend finds in a program (C[b, m, n] = Σ_k A[b, m, k] · B[b, k, n] with any
// strides), with the IR kernel's own statements as the epilogue.
//
// A workgroup of 256 lanes (4 wavefronts, 2 x 2) computes a BM x BN tile of C. The K loop walks
// 16-deep slices: each slice of A and B is loaded from global memory into registers one slice ahead,
// stored to LDS k-major (As[k][m], Bs[k][n]), and read back as MFMA operands: for the 32x32x2
// instruction lane l holds A[m0 + l % 32][k + l / 32] and B[k + l / 32][n0 + l % 32], and its 16
// accumulators are C[m0 + 8 (v / 4) + 4 (l / 32) + v % 4][n0 + l % 32], v = 0..15. Two LDS
// buffers and one barrier per slice.
//
// Loads are float4 along whichever index is contiguous in memory (k, or m / n); an operand with
// neither contiguous is loaded element by element. Out-of-range rows, columns and k are zero.
//
// Products with few output tiles and a long K (a batch-256 layer: 256 x 1024 outputs, K = 1024) use
// anvil_mm_tile_ksplit instead: the workgroup's four wavefronts share one 32 x 32 tile and split K
// four ways, and their partial tiles are added through LDS. (Splitting K across workgroups would
// need a device-scope release fence per workgroup to publish partial tiles, which on a part whose
// L2 caches are per XCD means writing back the L2: far slower than the product itself.)
#pragma once
#ifndef ANVIL_EMULATE

typedef float anvil_f32x16 __attribute__((ext_vector_type(16)));
typedef float anvil_f32x4 __attribute__((ext_vector_type(4)));

#define ANVIL_MM_BK 16
#define ANVIL_LD_KC 0        // contiguous along k
#define ANVIL_LD_RC 1        // contiguous along the row / column index (m for A, n for B)
#define ANVIL_LD_ANY 2       // neither: one element at a time

// One operand's BK x BT slice (T = BM for A, BN for B) between global memory, registers and LDS,
// moved by NT cooperating lanes (a workgroup, or one wavefront). `rs` = stride of the row/column
// index, `ks` = stride of k, in elements.
template <int BT, int MODE, int NT>
struct anvil_slice {
    static constexpr int PER = BT * ANVIL_MM_BK / NT;            // elements per lane
    static constexpr int LD = BT + 4;                            // LDS row length (k-major)
    float r[PER];

    template <class OP>
    __device__ __forceinline__ void load(const float *__restrict__ p, long long rs, long long ks, int t0, int tmax,
                                         int k0, int kend, OP op, int tid) {
        if (MODE == ANVIL_LD_KC) {                               // float4 along k
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + NT * q, tl = idx >> 2, kl = (idx & 3) * 4;
                const int t = t0 + tl, k = k0 + kl;
                anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (t < tmax && k < kend) v = *(const anvil_f32x4 *)(p + (long long)t * rs + k);
                r[4 * q + 0] = (t < tmax && k + 0 < kend) ? op(v.x) : 0.f;
                r[4 * q + 1] = (t < tmax && k + 1 < kend) ? op(v.y) : 0.f;
                r[4 * q + 2] = (t < tmax && k + 2 < kend) ? op(v.z) : 0.f;
                r[4 * q + 3] = (t < tmax && k + 3 < kend) ? op(v.w) : 0.f;
            }
        } else if (MODE == ANVIL_LD_RC) {                        // float4 along the tile index
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + NT * q, kl = idx / (BT / 4), tl = (idx % (BT / 4)) * 4;
                const int t = t0 + tl, k = k0 + kl;
                anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (t < tmax && k < kend) v = *(const anvil_f32x4 *)(p + (long long)k * ks + t);
                r[4 * q + 0] = (t + 0 < tmax && k < kend) ? op(v.x) : 0.f;
                r[4 * q + 1] = (t + 1 < tmax && k < kend) ? op(v.y) : 0.f;
                r[4 * q + 2] = (t + 2 < tmax && k < kend) ? op(v.z) : 0.f;
                r[4 * q + 3] = (t + 3 < tmax && k < kend) ? op(v.w) : 0.f;
            }
        } else {
#pragma unroll
            for (int q = 0; q < PER; q++) {
                const int idx = tid + NT * q, tl = idx % BT, kl = idx / BT;
                const int t = t0 + tl, k = k0 + kl;
                r[q] = (t < tmax && k < kend) ? op(p[(long long)t * rs + (long long)k * ks]) : 0.f;
            }
        }
    }

    __device__ __forceinline__ void store(float *__restrict__ s, int tid) const {
        if (MODE == ANVIL_LD_KC) {
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + NT * q, tl = idx >> 2, kl = (idx & 3) * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) s[(kl + i) * LD + tl] = r[4 * q + i];
            }
        } else if (MODE == ANVIL_LD_RC) {
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + NT * q, kl = idx / (BT / 4), tl = (idx % (BT / 4)) * 4;
                anvil_f32x4 v = {r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]};
                *(anvil_f32x4 *)(s + kl * LD + tl) = v;
            }
        } else {
#pragma unroll
            for (int q = 0; q < PER; q++) {
                const int idx = tid + NT * q, tl = idx % BT, kl = idx / BT;
                s[kl * LD + tl] = r[q];
            }
        }
    }
};

struct anvil_identity_op {
    __device__ __forceinline__ float operator()(float x) const { return x; }
};

// The accumulators of one wavefront: TM x TN tiles of 32 x 32.
template <int TM, int TN>
struct anvil_mm_acc {
    anvil_f32x16 c[TM][TN];
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) c[i][j][v] = 0.f;
    }
};

// C tile (m0, n0) over k in [kbeg, kend): A(m, k) = a[m * a_rs + k * a_ks], B(k, n) = b[k * b_ks + n * b_rs].
template <int BM, int BN, int AMODE, int BMODE, class OPA, class OPB>
__device__ __forceinline__ void anvil_mm_tile(anvil_mm_acc<BM / 64, BN / 64> &acc,
                                              const float *__restrict__ a, long long a_rs, long long a_ks,
                                              const float *__restrict__ b, long long b_rs, long long b_ks,
                                              int M, int N, int m0, int n0, int kbeg, int kend, OPA opa, OPB opb) {
    constexpr int TM = BM / 64, TN = BN / 64;
    __shared__ float As[2][ANVIL_MM_BK * (BM + 4)];
    __shared__ float Bs[2][ANVIL_MM_BK * (BN + 4)];
    anvil_slice<BM, AMODE, 256> sa;
    anvil_slice<BN, BMODE, 256> sb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
    const int lr = lane & 31, lk = lane >> 5;
    acc.zero();
    if (kbeg >= kend) return;
    sa.load(a, a_rs, a_ks, m0, M, kbeg, kend, opa, tid);
    sb.load(b, b_rs, b_ks, n0, N, kbeg, kend, opb, tid);
    sa.store(As[0], tid);
    sb.store(Bs[0], tid);
    __syncthreads();
    int buf = 0;
    for (int k0 = kbeg; k0 < kend; k0 += ANVIL_MM_BK) {
        const int next = k0 + ANVIL_MM_BK;
        if (next < kend) {
            sa.load(a, a_rs, a_ks, m0, M, next, kend, opa, tid);
            sb.load(b, b_rs, b_ks, n0, N, next, kend, opb, tid);
        }
        const float *as = As[buf];
        const float *bs = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < ANVIL_MM_BK; kk += 2) {
            float fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) fa[i] = as[(kk + lk) * (BM + 4) + wm + 32 * i + lr];
#pragma unroll
            for (int j = 0; j < TN; j++) fb[j] = bs[(kk + lk) * (BN + 4) + wn + 32 * j + lr];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc.c[i][j], 0, 0, 0);
        }
        if (next < kend) {
            sa.store(As[buf ^ 1], tid);
            sb.store(Bs[buf ^ 1], tid);
        }
        __syncthreads();
        buf ^= 1;
    }
}

// K split inside one workgroup: the 4 wavefronts all compute the same (32 TM) x (32 TN) tile, wave w
// over the 16-deep k slices w, w + 4, w + 8, ... (every wave runs the same number of rounds; a
// slice past the end loads zeros). Each wave stages its own slices in its own LDS region. At the
// end the four partial tiles are added through LDS in wave order (a fixed order: the result does
// not depend on timing) and wave w keeps accumulators 4w .. 4w+3 of every 32x32 sub-tile in `out`.
template <int TM, int TN, int AMODE, int BMODE, class OPA, class OPB>
__device__ __forceinline__ void anvil_mm_tile_ksplit(float (&out)[TM][TN][4],
                                                     const float *__restrict__ a, long long a_rs, long long a_ks,
                                                     const float *__restrict__ b, long long b_rs, long long b_ks,
                                                     int M, int N, int m0, int n0, int kbeg, int kend, OPA opa, OPB opb) {
    constexpr int BM = 32 * TM, BN = 32 * TN;
    constexpr int SA = ANVIL_MM_BK * (BM + 4), SB = ANVIL_MM_BK * (BN + 4);
    static_assert(4 * TM * TN * 16 * 64 <= 4 * 2 * (SA + SB), "partial tiles must fit in the staging LDS");
    __shared__ float lds[4 * 2 * (SA + SB)];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lr = lane & 31, lk = lane >> 5;
    float *As = lds + w * 2 * (SA + SB);
    float *Bs = As + 2 * SA;
    anvil_slice<BM, AMODE, 64> sa;
    anvil_slice<BN, BMODE, 64> sb;
    anvil_mm_acc<TM, TN> acc;
    acc.zero();
    const int slices = (kend - kbeg + ANVIL_MM_BK - 1) / ANVIL_MM_BK;
    const int rounds = (slices + 3) / 4;
    int k0 = kbeg + ANVIL_MM_BK * w;
    sa.load(a, a_rs, a_ks, m0, M, k0, kend, opa, lane);
    sb.load(b, b_rs, b_ks, n0, N, k0, kend, opb, lane);
    sa.store(As, lane);
    sb.store(Bs, lane);
    __syncthreads();
    int buf = 0;
    for (int r = 0; r < rounds; r++) {
        const int kn = k0 + 4 * ANVIL_MM_BK;
        const bool more = r + 1 < rounds;
        if (more) {
            sa.load(a, a_rs, a_ks, m0, M, kn, kend, opa, lane);
            sb.load(b, b_rs, b_ks, n0, N, kn, kend, opb, lane);
        }
        const float *as = As + buf * SA;
        const float *bs = Bs + buf * SB;
#pragma unroll
        for (int kk = 0; kk < ANVIL_MM_BK; kk += 2) {
            float fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) fa[i] = as[(kk + lk) * (BM + 4) + 32 * i + lr];
#pragma unroll
            for (int j = 0; j < TN; j++) fb[j] = bs[(kk + lk) * (BN + 4) + 32 * j + lr];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc.c[i][j], 0, 0, 0);
        }
        if (more) {
            sa.store(As + (buf ^ 1) * SA, lane);
            sb.store(Bs + (buf ^ 1) * SB, lane);
        }
        __syncthreads();
        buf ^= 1;
        k0 = kn;
    }
    // the four partial tiles, through LDS (the staging area is free now): part[w][i][j][v][lane]
    float *part = lds;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) part[(((w * TM + i) * TN + j) * 16 + v) * 64 + lane] = acc.c[i][j][v];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float s = 0.f;
#pragma unroll
                for (int src = 0; src < 4; src++) s += part[(((src * TM + i) * TN + j) * 16 + 4 * w + q) * 64 + lane];
                out[i][j][q] = s;
            }
}

#endif
