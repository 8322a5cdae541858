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
typedef float anvil_f32x2 __attribute__((ext_vector_type(2)));

#ifndef ANVIL_MM_BK
#define ANVIL_MM_BK 16       // k depth of the LDS-staged tile schedule's slices
#endif
#define ANVIL_LD_KC 0        // contiguous along k
#define ANVIL_LD_RC 1        // contiguous along the row / column index (m for A, n for B)
#define ANVIL_LD_ANY 2       // neither: one element at a time
#define ANVIL_LD_KT 3        // one element at a time, where each of 4 consecutive k starts is read from
                             // a table (k over variables whose strides do not line up: a convolution's
                             // input read as c, u, v while the weights run linearly over them)

typedef int anvil_i32x4 __attribute__((ext_vector_type(4)));

// XCD-aware tile order. Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2: tile (tx, ty) of a tn x tm grid for linear id L is chosen so that the ids one XCD receives
// (L mod 8 = x) cover one contiguous run p of tiles, and runs are walked in groups of G tile rows,
// column by column: an XCD's tiles then share few row panels of A and column panels of B.
__device__ __forceinline__ int anvil_run_of(int L, int n) {
    // the position in 0 .. n - 1 of linear id L when the ids of XCD x = L mod 8 take one contiguous
    // run of positions (runs of n / 8, the first n mod 8 of them one longer)
    const int q = n / 8, rem = n % 8;
    return (L % 8) * q + min(L % 8, rem) + L / 8;
}

__device__ __forceinline__ void anvil_tile_of(int L, int tn, int tm, int G, int &tx, int &ty) {
    const int n = tn * tm, q = n / 8, rem = n % 8;
    const int x = L % 8, r = L / 8;
    const int p = x * q + min(x, rem) + r;
    const int group = p / (G * tn), within = p % (G * tn);
    const int gm = min(G, tm - group * G);
    ty = group * G + within % gm;
    tx = within / gm;
}

// The offsets of k .. k + 3 (k a multiple of 4) in an operand: kf(k) + s·ks, or four table entries.
template <int MODE, class KF>
__device__ __forceinline__ void anvil_koffs(KF kf, int k, long long ks, long long (&o)[4]) {
    if constexpr (MODE == ANVIL_LD_KT) {
        kf.quad(k, o);
    } else {
        const long long b = kf(k);
        o[0] = b;
        o[1] = b + ks;
        o[2] = b + 2 * ks;
        o[3] = b + 3 * ks;
    }
}

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

// K split inside one workgroup: its W wavefronts all compute the same (32 TM) x (32 TN) tile, wave w
// over the w-th of W equal shares of K. The waves share no operands, so each loads its MFMA operands straight
// from global memory into registers, U chunks of 8 k at a time, one batch ahead of the MFMAs: lane
// l (row or column r = l % 32, half h = l / 32) holds element k0 + 4h + s of its row of A and of its
// column of B for s = 0..3, and MFMA s of the chunk takes slot s (any assignment of k values to
// MFMA k slots gives the same sum, as long as A and B agree). A k-contiguous operand is one float4
// per lane and chunk; otherwise 4 loads, coalesced across the 32 lanes when the row index is
// contiguous. At the end the W partial tiles are added through LDS in wave order (a fixed order:
// the result does not depend on timing) and wave w keeps accumulators (16/W) w .. (16/W)(w+1) - 1
// of every 32x32 sub-tile in `out`.
template <int MODE, class OP>
__device__ __forceinline__ void anvil_chunk_load(float (&r)[4], const float *__restrict__ p, long long rs, long long ks,
                                                 int t, int tmax, int k, int kend, OP op) {
    if (MODE == ANVIL_LD_KC) {
        anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (t < tmax && k < kend) v = *(const anvil_f32x4 *)(p + (long long)t * rs + k);
        r[0] = (t < tmax && k + 0 < kend) ? op(v.x) : 0.f;
        r[1] = (t < tmax && k + 1 < kend) ? op(v.y) : 0.f;
        r[2] = (t < tmax && k + 2 < kend) ? op(v.z) : 0.f;
        r[3] = (t < tmax && k + 3 < kend) ? op(v.w) : 0.f;
    } else {
#pragma unroll
        for (int s = 0; s < 4; s++)
            r[s] = (t < tmax && k + s < kend) ? op(p[(long long)t * rs + (long long)(k + s) * ks]) : 0.f;
    }
}

template <int TM, int TN, int AMODE, int BMODE, int U, class OPA, class OPB>
__device__ __forceinline__ void anvil_mm_wave(anvil_mm_acc<TM, TN> &acc,
                                              const float *__restrict__ a, long long a_rs, long long a_ks,
                                              const float *__restrict__ b, long long b_rs, long long b_ks,
                                              int M, int N, int m0, int n0, int kbeg, int kend, OPA opa, OPB opb) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    float a0[U][TM][4], b0[U][TN][4], a1[U][TM][4], b1[U][TN][4];
    constexpr int STEP = 8 * U;
    acc.zero();
#define ANVIL_MM_LOAD(AR, BR, KB)                                                                          \
    _Pragma("unroll") for (int u = 0; u < U; u++) {                                                        \
        _Pragma("unroll") for (int i = 0; i < TM; i++)                                                     \
            anvil_chunk_load<AMODE>(AR[u][i], a, a_rs, a_ks, m0 + 32 * i + r, M, (KB) + 8 * u + 4 * h, kend, opa); \
        _Pragma("unroll") for (int j = 0; j < TN; j++)                                                     \
            anvil_chunk_load<BMODE>(BR[u][j], b, b_rs, b_ks, n0 + 32 * j + r, N, (KB) + 8 * u + 4 * h, kend, opb); \
    }
#define ANVIL_MM_MFMA(AR, BR)                                                                              \
    _Pragma("unroll") for (int u = 0; u < U; u++)                                                          \
        _Pragma("unroll") for (int s = 0; s < 4; s++)                                                      \
            _Pragma("unroll") for (int i = 0; i < TM; i++)                                                 \
                _Pragma("unroll") for (int j = 0; j < TN; j++)                                             \
                    acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(AR[u][i][s], BR[u][j][s], acc.c[i][j], 0, 0, 0);
    ANVIL_MM_LOAD(a0, b0, kbeg)
    for (int kb = kbeg; kb < kend; kb += 2 * STEP) {
        ANVIL_MM_LOAD(a1, b1, kb + STEP)
        ANVIL_MM_MFMA(a0, b0)
        if (kb + STEP >= kend) break;                  // the second batch is past the end: all zeros
        ANVIL_MM_LOAD(a0, b0, kb + 2 * STEP)
        ANVIL_MM_MFMA(a1, b1)
    }
#undef ANVIL_MM_LOAD
#undef ANVIL_MM_MFMA
}

template <int W, int TM, int TN, int AMODE, int BMODE, int U, class OPA, class OPB>
__device__ __forceinline__ void anvil_mm_tile_ksplit(float (&out)[TM][TN][16 / W],
                                                     const float *__restrict__ a, long long a_rs, long long a_ks,
                                                     const float *__restrict__ b, long long b_rs, long long b_ks,
                                                     int M, int N, int m0, int n0, int kbeg, int kend, OPA opa, OPB opb) {
    constexpr int PER = 16 / W;                                       // accumulators each wave finishes
    __shared__ float part[W * TM * TN * 16 * 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int share = ((kend - kbeg + W - 1) / W + 7) / 8 * 8;        // a multiple of the 8-k chunk
    const int kb = kbeg + w * share, ke = min(kend, kb + share);
    anvil_mm_acc<TM, TN> acc;
    anvil_mm_wave<TM, TN, AMODE, BMODE, U>(acc, a, a_rs, a_ks, b, b_rs, b_ks, M, N, m0, n0, kb, ke, opa, opb);
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
            for (int q = 0; q < PER; q++) {
                float s = 0.f;
#pragma unroll
                for (int src = 0; src < W; src++) s += part[(((src * TM + i) * TN + j) * 16 + PER * w + q) * 64 + lane];
                out[i][j][q] = s;
            }
}

// The same K split with a software pipeline (K a multiple of 8G): the K range is cut into C chunks
// of 8G k, NCH consecutive ones per wave (the last busy wave may have fewer, later waves none). A
// wave keeps D chunks of operands in flight: it waits only for the oldest, runs its 4G MFMAs, and
// reuses those registers for the chunk D ahead, so the matrix cores start on the first data to
// arrive instead of after the last. In a chunk, lane (r, h) holds k0 + 4G·h + s (s < 4G) of its
// row r, and MFMA s pairs k0 + s with k0 + 4G + s: an operand contiguous in k is read with G
// 16-byte loads per lane, so with G = 4 the two half-waves cover 128 bytes, a whole cache line, of
// each of the 32 rows (G = 1: a quarter line per row and load, the other quarters coming in later
// chunks after the line may have left the L1). The chunk loop is unrolled (NCH is a compile-time constant):
// straight-line code, where the compiler's wait counts are exact. Rows and columns past M / N are
// zero (CHKM, CHKN: the tile may cross the edge); k is always in range. Where row (column) t of
// an operand starts is arow(t) (brow(t)): t times its stride, or, for rows picked through an index
// array (a shuffled batch, X[perm[i]]), that row's offset; each lane computes its rows' once. Where
// k-index k starts is ak(k) (bk(k)): k times the stride, or, when K runs over several loop
// variables (a weight gradient summed over the batch and the positions of a convolution), their
// offsets; 4 consecutive k are a_ks (b_ks) apart. The workgroup covers k in [kbeg, kbeg + K).
template <int MODE, bool CHK>
__device__ __forceinline__ void anvil_chunk_load_k(float (&r)[4], const float *__restrict__ p, long long toff,
                                                   const long long (&ko)[4], int t, int tmax, bool ok = true) {
    if ((CHK && t >= tmax) || !ok) {
        r[0] = r[1] = r[2] = r[3] = 0.f;
        return;
    }
    if (MODE == ANVIL_LD_KC) {
        const anvil_f32x4 v = *(const anvil_f32x4 *)(p + toff + ko[0]);
        r[0] = v.x;
        r[1] = v.y;
        r[2] = v.z;
        r[3] = v.w;
    } else {
#pragma unroll
        for (int s = 0; s < 4; s++) r[s] = p[toff + ko[s]];
    }
}

// Which (row, k) operand elements exist: all of them, unless a product reads a window of its
// operand that may hang over the edge (a convolution's input gradient: dY[y - u]); the 4
// consecutive k a lane loads at once share the answer.
struct anvil_all_pred {
    __device__ __forceinline__ bool operator()(int, int) const { return true; }
};

template <int TM, int TN, int AMODE, int BMODE, int NCH, int D, bool CHKM, bool CHKN, bool FULL, int G, int CH,
          class AK, class BK, class OPA, class OPB, class APRED, class BPRED>
__device__ __forceinline__ void anvil_mm_wave_kpipe(anvil_mm_acc<TM, TN> &acc,
                                                    const float *__restrict__ a, const long long (&ao)[TM], AK ak,
                                                    long long a_ks, const float *__restrict__ b,
                                                    const long long (&bo)[TN], BK bk, long long b_ks,
                                                    int M, int N, int m0, int n0, int c0, int n, OPA opa, OPB opb,
                                                    APRED apred, BPRED bpred) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    float ab[D][TM][4 * G], bb[D][TN][4 * G];
#define ANVIL_KP_LOAD(d, c)                                                                                \
    if (FULL || (c) < n) {                                                                                 \
        _Pragma("unroll") for (int g = 0; g < G; g++) {                                                    \
            const int k_ = 8 * G * (c0 + (c)) + 4 * G * h + 4 * g;                                        \
            long long ka_[4], kb_[4];                                                                      \
            anvil_koffs<AMODE>(ak, k_, a_ks, ka_);                                                         \
            anvil_koffs<BMODE>(bk, k_, b_ks, kb_);                                                         \
            _Pragma("unroll") for (int i = 0; i < TM; i++)                                                 \
                anvil_chunk_load_k<AMODE, CHKM>(*reinterpret_cast<float(*)[4]>(&ab[d][i][4 * g]), a, ao[i], \
                                                ka_, m0 + 32 * i + r, M, apred(m0 + 32 * i + r, k_));       \
            _Pragma("unroll") for (int j = 0; j < TN; j++)                                                 \
                anvil_chunk_load_k<BMODE, CHKN>(*reinterpret_cast<float(*)[4]>(&bb[d][j][4 * g]), b, bo[j], \
                                                kb_, n0 + 32 * j + r, N, bpred(n0 + 32 * j + r, k_));       \
        }                                                                                                  \
    }
#pragma unroll
    for (int c = 0; c < D; c++) ANVIL_KP_LOAD(c, c)
    __builtin_amdgcn_sched_barrier(0);          // every load of the prologue is issued before the first MFMA
    // CH independent accumulator chains: MFMA s of a chunk adds into chain s % CH (a dependent MFMA
    // waits for its predecessor's result; two chains let the matrix core overlap them)
    anvil_mm_acc<TM, TN> acc2;
    if (CH > 1) acc2.zero();
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        if (FULL || c < n) {
#pragma unroll
            for (int s = 0; s < 4 * G; s++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        if (CH > 1 && (s & 1))
                            acc2.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(opa(ab[c % D][i][s]), opb(bb[c % D][j][s]),
                                                                                acc2.c[i][j], 0, 0, 0);
                        else
                            acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(opa(ab[c % D][i][s]), opb(bb[c % D][j][s]),
                                                                               acc.c[i][j], 0, 0, 0);
                    }
        }
        if (c + D < NCH) ANVIL_KP_LOAD(c % D, c + D)
        __builtin_amdgcn_sched_barrier(0);
    }
    if (CH > 1) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc.c[i][j] += acc2.c[i][j];
    }
#undef ANVIL_KP_LOAD
}

template <int W, int TM, int TN, int AMODE, int BMODE, int NCH, int D, bool CHKM, bool CHKN, int G = 1, int CH = 1,
          class AROW, class BROW, class AK, class BK, class OPA, class OPB, class APRED = anvil_all_pred,
          class BPRED = anvil_all_pred>
__device__ __forceinline__ void anvil_mm_tile_kpipe(float *__restrict__ part, float (&out)[TM][TN][16 / W],
                                                    const float *__restrict__ a, AROW arow, AK ak, long long a_ks,
                                                    const float *__restrict__ b, BROW brow, BK bk, long long b_ks,
                                                    int M, int N, int m0, int n0, int kbeg, int K, OPA opa, OPB opb,
                                                    APRED apred = APRED(), BPRED bpred = BPRED()) {
    // part: the caller's LDS for the wavefronts' partial tiles, W·TM·TN·16·64 floats (a side-by-side
    // launch gives all its parts the same array: a workgroup runs one part)
    constexpr int PER = 16 / W;
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);     // uniform: scalar branches
    const int c0 = kbeg / (8 * G) + w * NCH, n = min(NCH, max(0, (kbeg + K) / (8 * G) - c0));
    long long ao[TM], bo[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) ao[i] = (!CHKM || m0 + 32 * i + r < M) ? arow(m0 + 32 * i + r) : 0;
#pragma unroll
    for (int j = 0; j < TN; j++) bo[j] = (!CHKN || n0 + 32 * j + r < N) ? brow(n0 + 32 * j + r) : 0;
    anvil_mm_acc<TM, TN> acc;
    acc.zero();
    if (n == NCH)
        anvil_mm_wave_kpipe<TM, TN, AMODE, BMODE, NCH, D, CHKM, CHKN, true, G, CH>(acc, a, ao, ak, a_ks, b, bo, bk, b_ks, M,
                                                                               N, m0, n0, c0, n, opa, opb, apred, bpred);
    else if (n > 0)
        anvil_mm_wave_kpipe<TM, TN, AMODE, BMODE, NCH, D, CHKM, CHKN, false, G, CH>(acc, a, ao, ak, a_ks, b, bo, bk, b_ks, M,
                                                                                N, m0, n0, c0, n, opa, opb, apred, bpred);
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
            for (int q = 0; q < PER; q++) {
                float s = 0.f;
#pragma unroll
                for (int src = 0; src < W; src++) s += part[(((src * TM + i) * TN + j) * 16 + PER * w + q) * 64 + lane];
                out[i][j][q] = s;
            }
}

// A product whose A rows are computed in the kernel from the rows of another matrix (a layer
// norm's output, normalized from its input with row statistics) before the K split above runs on
// them. K is one whole row, split over the W wavefronts in NCH chunks of 8G k each; lane (r, h) of
// wavefront w holds, for tile row i, the k of the kpipe layout: x[i][(c·G + g)·4 + s] is element
// k = 8G(w·NCH + c) + 4G·h + 4g + s of row m0 + 32i + r. The raw row elements are loaded
// (anvil_rowpro_load), the generated code turns them into the A values in place (row sums through
// anvil_rowpro_sum), and anvil_mm_tile_kpipe_areg runs the products with A from those registers
// and only B loaded, D chunks in flight.
template <int TM, int NCH, int G, bool CHKM>
__device__ __forceinline__ void anvil_rowpro_load(float (&x)[TM][NCH * 4 * G], const float *__restrict__ p,
                                                  long long rs, int m0, int M) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int row = m0 + 32 * i + r;
#pragma unroll
        for (int c = 0; c < NCH; c++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                const int k = 8 * G * (w * NCH + c) + 4 * G * h + 4 * g;
                anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (!CHKM || row < M) v = *(const anvil_f32x4 *)(p + (long long)row * rs + k);
                x[i][(c * G + g) * 4 + 0] = v.x;
                x[i][(c * G + g) * 4 + 1] = v.y;
                x[i][(c * G + g) * 4 + 2] = v.z;
                x[i][(c * G + g) * 4 + 3] = v.w;
            }
    }
}

// The k index of element q of the lane's row registers (the layout above).
template <int NCH, int G>
__device__ __forceinline__ int anvil_rowpro_k(int q) {
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = q / (4 * G), g = (q / 4) % G, s = q % 4;
    return 8 * G * (w * NCH + c) + 4 * G * h + 4 * g + s;
}

// Each lane's partial sums of its rows (p[i], the lane's terms of row m0 + 32i + r) become the whole
// rows' sums: the two half-waves added, then the W wavefronts' partials in wavefront order.
// lds: W·TM·32 floats.
template <int W, int TM>
__device__ __forceinline__ void anvil_rowpro_sum(float (&p)[TM], float *__restrict__ lds) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        p[i] += __shfl_xor(p[i], 32, 64);
        if (h == 0) lds[(w * TM + i) * 32 + r] = p[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; i++) {
        float s = lds[i * 32 + r];
#pragma unroll
        for (int src = 1; src < W; src++) s += lds[(src * TM + i) * 32 + r];
        p[i] = s;
    }
    __syncthreads();
}

template <int W, int TM, int TN, int BMODE, int NCH, int D, bool CHKN, int G, int CH, class BROW, class BK, class OPB>
__device__ __forceinline__ void anvil_mm_tile_kpipe_areg(float *__restrict__ part, float (&out)[TM][TN][16 / W],
                                                         const float (&xa)[TM][NCH * 4 * G],
                                                         const float *__restrict__ b, BROW brow, BK bk, long long b_ks,
                                                         int N, int n0, OPB opb) {
    constexpr int PER = 16 / W;
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c0 = w * NCH;
    long long bo[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) bo[j] = (!CHKN || n0 + 32 * j + r < N) ? brow(n0 + 32 * j + r) : 0;
    anvil_mm_acc<TM, TN> acc, acc2;
    acc.zero();
    if (CH > 1) acc2.zero();
    float bb[D][TN][4 * G];
    anvil_all_pred bpred;
#define ANVIL_KPA_LOAD(d, c)                                                                               \
    _Pragma("unroll") for (int g = 0; g < G; g++) {                                                        \
        const int k_ = 8 * G * (c0 + (c)) + 4 * G * h + 4 * g;                                            \
        long long kb_[4];                                                                                  \
        anvil_koffs<BMODE>(bk, k_, b_ks, kb_);                                                             \
        _Pragma("unroll") for (int j = 0; j < TN; j++)                                                     \
            anvil_chunk_load_k<BMODE, CHKN>(*reinterpret_cast<float(*)[4]>(&bb[d][j][4 * g]), b, bo[j], kb_, \
                                            n0 + 32 * j + r, N, bpred(n0 + 32 * j + r, k_));               \
    }
#pragma unroll
    for (int c = 0; c < D; c++) ANVIL_KPA_LOAD(c, c)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
#pragma unroll
        for (int s = 0; s < 4 * G; s++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    if (CH > 1 && (s & 1))
                        acc2.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[i][c * 4 * G + s], opb(bb[c % D][j][s]),
                                                                            acc2.c[i][j], 0, 0, 0);
                    else
                        acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[i][c * 4 * G + s], opb(bb[c % D][j][s]),
                                                                           acc.c[i][j], 0, 0, 0);
                }
        if (c + D < NCH) ANVIL_KPA_LOAD(c % D, c + D)
        __builtin_amdgcn_sched_barrier(0);
    }
#undef ANVIL_KPA_LOAD
    if (CH > 1) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc.c[i][j] += acc2.c[i][j];
    }
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
            for (int q = 0; q < PER; q++) {
                float s = 0.f;
#pragma unroll
                for (int src = 0; src < W; src++) s += part[(((src * TM + i) * TN + j) * 16 + PER * w + q) * 64 + lane];
                out[i][j][q] = s;
            }
}

// The K split with operands staged through LDS: the workgroup's 256 lanes load each KC-deep chunk
// of A (32 rows) and B (32 columns) with 16-byte loads along whichever index is contiguous in
// memory (a wavefront's load covers a few whole cache lines, where loading MFMA operands straight
// into registers touches one line per row), store it to LDS k-major, and each wavefront runs the
// MFMAs of its quarter of the chunk's k from LDS. The next chunk is loaded into registers while the
// current one is multiplied; two LDS buffers, one barrier per chunk. The four partial tiles are
// added through LDS in wave order at the end, as in anvil_mm_tile_ksplit.
template <int MODE, int KC, bool CHKT, int LD>
struct anvil_slab {
    // one operand's 32 x KC chunk: element (t, k) at p[t * rs + k * ks]
    static constexpr int PER = 32 * KC / 256;                       // elements per lane
    float r[PER];

    template <class OP>
    __device__ __forceinline__ void load(const float *__restrict__ p, long long rs, long long ks, int t0, int tmax,
                                         int k0, int kend, OP op, int tid) {
        if (MODE == ANVIL_LD_KC) {                                  // 16 bytes along k
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + 256 * q, tl = idx / (KC / 4), kl = (idx % (KC / 4)) * 4;
                const int t = t0 + tl, k = k0 + kl;
                anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if ((!CHKT || t < tmax) && k + 3 < kend) {
                    v = *(const anvil_f32x4 *)(p + (long long)t * rs + k);
                } else if (!CHKT || t < tmax) {
                    if (k + 0 < kend) v.x = p[(long long)t * rs + k + 0];
                    if (k + 1 < kend) v.y = p[(long long)t * rs + k + 1];
                    if (k + 2 < kend) v.z = p[(long long)t * rs + k + 2];
                }
                r[4 * q + 0] = op(v.x);
                r[4 * q + 1] = op(v.y);
                r[4 * q + 2] = op(v.z);
                r[4 * q + 3] = op(v.w);
            }
        } else if (MODE == ANVIL_LD_RC) {                           // 16 bytes along the tile index
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + 256 * q, kl = idx / 8, tl = (idx % 8) * 4;
                const int t = t0 + tl, k = k0 + kl;
                anvil_f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (k < kend) {
                    if (!CHKT || t + 3 < tmax) {
                        v = *(const anvil_f32x4 *)(p + (long long)k * ks + t);
                    } else {
                        if (t + 0 < tmax) v.x = p[(long long)k * ks + t + 0];
                        if (t + 1 < tmax) v.y = p[(long long)k * ks + t + 1];
                        if (t + 2 < tmax) v.z = p[(long long)k * ks + t + 2];
                    }
                }
                r[4 * q + 0] = op(v.x);
                r[4 * q + 1] = op(v.y);
                r[4 * q + 2] = op(v.z);
                r[4 * q + 3] = op(v.w);
            }
        } else {
#pragma unroll
            for (int q = 0; q < PER; q++) {
                const int idx = tid + 256 * q, tl = idx % 32, kl = idx / 32;
                const int t = t0 + tl, k = k0 + kl;
                r[q] = ((!CHKT || t < tmax) && k < kend) ? op(p[(long long)t * rs + (long long)k * ks]) : 0.f;
            }
        }
    }

    // k-major in LDS: s[k * LD + t]
    __device__ __forceinline__ void store(float *__restrict__ s, int tid) const {
        if (MODE == ANVIL_LD_KC) {
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + 256 * q, tl = idx / (KC / 4), kl = (idx % (KC / 4)) * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) s[(kl + i) * LD + tl] = r[4 * q + i];
            }
        } else if (MODE == ANVIL_LD_RC) {
#pragma unroll
            for (int q = 0; q < PER / 4; q++) {
                const int idx = tid + 256 * q, kl = idx / 8, tl = (idx % 8) * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) s[kl * LD + tl + i] = r[4 * q + i];
            }
        } else {
#pragma unroll
            for (int q = 0; q < PER; q++) {
                const int idx = tid + 256 * q, tl = idx % 32, kl = idx / 32;
                s[kl * LD + tl] = r[q];
            }
        }
    }
};

template <int AMODE, int BMODE, int KC, bool CHKM, bool CHKN, class OPA, class OPB>
__device__ __forceinline__ void anvil_mm_tile_kslab(float (&out)[1][1][4],
                                                    const float *__restrict__ a, long long a_rs, long long a_ks,
                                                    const float *__restrict__ b, long long b_rs, long long b_ks,
                                                    int M, int N, int m0, int n0, int K, OPA opa, OPB opb) {
    constexpr int LD = 33;                                          // odd: k-major stores spread over banks
    __shared__ float As[2][KC * LD];
    __shared__ float Bs[2][KC * LD];
    __shared__ float part[4 * 16 * 64];
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    anvil_slab<AMODE, KC, CHKM, LD> sa;
    anvil_slab<BMODE, KC, CHKN, LD> sb;
    anvil_mm_acc<1, 1> acc;
    acc.zero();
    sa.load(a, a_rs, a_ks, m0, M, 0, K, opa, tid);
    sb.load(b, b_rs, b_ks, n0, N, 0, K, opb, tid);
    sa.store(As[0], tid);
    sb.store(Bs[0], tid);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < K; k0 += KC) {
        const int next = k0 + KC;
        if (next < K) {
            sa.load(a, a_rs, a_ks, m0, M, next, K, opa, tid);
            sb.load(b, b_rs, b_ks, n0, N, next, K, opb, tid);
        }
        const float *as = As[buf] + (KC / 4) * w * LD;
        const float *bs = Bs[buf] + (KC / 4) * w * LD;
#pragma unroll
        for (int kk = 0; kk < KC / 4; kk += 2)
            acc.c[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(as[(kk + h) * LD + r], bs[(kk + h) * LD + r],
                                                               acc.c[0][0], 0, 0, 0);
        if (next < K) {
            sa.store(As[buf ^ 1], tid);
            sb.store(Bs[buf ^ 1], tid);
        }
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int v = 0; v < 16; v++) part[(w * 16 + v) * 64 + lane] = acc.c[0][0][v];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float s = 0.f;
#pragma unroll
        for (int src = 0; src < 4; src++) s += part[(src * 16 + 4 * w + q) * 64 + lane];
        out[0][0][q] = s;
    }
}

// Attention without the score matrix: O[b] = softmax(scale · Q[b] K[b]ᵀ) V[b], rows of Q in 32-query
// tiles, one tile per workgroup whose four wavefronts each take a quarter of the keys (32 at a time)
// and are merged at the end (eight wavefronts, two per SIMD, measured 16 % slower). Everything is
// computed transposed, Sᵀ = K Qᵀ and Oᵀ = Vᵀ Pᵀ, so that lane l always holds query l % 32 (half
// h = l / 32): its running max and sum are lane-local, and the Sᵀ accumulators of lane l (keys 8(v/4) + 4h + v%4 of the tile) are exactly the Pᵀ operand
// lane l must supply to the next MFMAs, taking key slot h of MFMA v; the Vᵀ operand follows the same
// key order. Output rows d of the DT = D/32 Oᵀ tiles are interleaved, d = DT·i + j, so each lane
// loads DT consecutive floats of a V row at once. Per key tile: running max m, p = 2^(s - m) with s
// in base 2 (Q pre-scaled by scale · log2 e), l = l·c + Σp, O = O·c + Vᵀ p with c = 2^(m_old - m_new)
// (the online softmax; the reference exponentiates s·scale - max in base e after the full row: the
// same values up to rounding). O is rescaled only when some lane's maximum moved. The scaled query
// tile sits in LDS, shared by the four waves (registers go to K, V and the accumulators); the next
// tile's K and V rows are loaded while the current one is multiplied.
template <int D>
struct anvil_vec_of { typedef float type; };
template <> struct anvil_vec_of<64> { typedef float __attribute__((ext_vector_type(2))) type; };
template <> struct anvil_vec_of<128> { typedef anvil_f32x4 type; };

template <int D>
__device__ __forceinline__ void anvil_attention_tile(const float *__restrict__ q, const float *__restrict__ k,
                                                     const float *__restrict__ v, float *__restrict__ o,
                                                     float scale, int Lq, int Lk, int q0) {
    constexpr int DH = D / 2;                  // k-dimension per lane half in Sᵀ = K Qᵀ
    constexpr int DT = D / 32;                 // Oᵀ tiles
    typedef typename anvil_vec_of<D>::type vec;
    __shared__ float part[4][DT][16][64];
    __shared__ float stat[4][2][32];
    __shared__ float qsh[32][D + 4];            // the query tile, scaled: read by the four waves
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int per = Lk / 4, kb = w * per;
    // scores in base 2: Q is scaled once by scale · log2(e), and p = 2^(s - m) (v_exp_f32)
    const float qs = scale * 1.4426950408889634f;
    for (int i = threadIdx.x; i < 32 * D / 4; i += 256) {
        const int row = i / (D / 4), c4 = 4 * (i % (D / 4));
        const anvil_f32x4 x = *(const anvil_f32x4 *)(q + (long long)(q0 + row) * D + c4);
        qsh[row][c4] = x.x * qs; qsh[row][c4 + 1] = x.y * qs; qsh[row][c4 + 2] = x.z * qs; qsh[row][c4 + 3] = x.w * qs;
    }
    __syncthreads();
    const float *qrow = &qsh[r][DH * h];
    anvil_f32x16 oacc[DT];
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[j][e] = 0.f;
    float m = -__builtin_inff(), l = 0.f;
    float kr[DH];
    vec vr[16];
#define ANVIL_AT_LOADK(K0)                                                                                 \
    _Pragma("unroll") for (int s4 = 0; s4 < DH; s4 += 4) {                                                 \
        const anvil_f32x4 x = *(const anvil_f32x4 *)(k + (long long)((K0) + r) * D + DH * h + s4);          \
        kr[s4] = x.x; kr[s4 + 1] = x.y; kr[s4 + 2] = x.z; kr[s4 + 3] = x.w;                                 \
    }
#define ANVIL_AT_LOADV(K0)                                                                                 \
    _Pragma("unroll") for (int t = 0; t < 16; t++)                                                         \
        vr[t] = *(const vec *)(v + (long long)((K0) + 8 * (t >> 2) + 4 * h + (t & 3)) * D + DT * r);
    ANVIL_AT_LOADK(kb)
    ANVIL_AT_LOADV(kb)
    for (int k0 = kb; k0 < kb + per; k0 += 32) {
        anvil_f32x16 sacc;
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[e] = 0.f;
        int qo = 0;
        asm volatile("" : "+v"(qo));            // read Q from LDS here, each tile: not kept in registers
#pragma unroll
        for (int s = 0; s < DH; s++) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[s], qrow[s + qo], sacc, 0, 0, 0);
        if (k0 + 32 < kb + per) ANVIL_AT_LOADK(k0 + 32)
        float mx = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 16; e++) mx = fmaxf(mx, sacc[e]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(m, mx);
        const float c = (mn == -__builtin_inff()) ? 1.f : __builtin_amdgcn_exp2f(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            sacc[e] = __builtin_amdgcn_exp2f(sacc[e] - mn);
            ps += sacc[e];
        }
        ps += __shfl_xor(ps, 32, 64);
        l = l * c + ps;
        m = mn;
        if (!__all(c == 1.f)) {                 // a new maximum somewhere in the wave: rescale O
#pragma unroll
            for (int j = 0; j < DT; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) oacc[j][e] *= c;
        }
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const float *vt = (const float *)&vr[t];
#pragma unroll
            for (int j = 0; j < DT; j++) oacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt[j], sacc[t], oacc[j], 0, 0, 0);
        }
        if (k0 + 32 < kb + per) ANVIL_AT_LOADV(k0 + 32)
    }
#undef ANVIL_AT_LOADK
#undef ANVIL_AT_LOADV
    // merge the four waves' (m, l, O) for each query, wave j finishing Oᵀ tile j (DT <= 4 ... DT tiles
    // split over the waves)
    if (h == 0) {
        stat[w][0][r] = m;
        stat[w][1][r] = l;
    }
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) part[w][j][e][lane] = oacc[j][e];
    __syncthreads();
    float M = stat[0][0][r];
#pragma unroll
    for (int x = 1; x < 4; x++) M = fmaxf(M, stat[x][0][r]);
    float f[4], L = 0.f;
#pragma unroll
    for (int x = 0; x < 4; x++) {
        const float mx = stat[x][0][r];
        f[x] = (mx == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(mx - M);
        L += f[x] * stat[x][1][r];
    }
    const float inv = 1.f / L;
    for (int j = w; j < DT; j += 4) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            float acc = 0.f;
#pragma unroll
            for (int x = 0; x < 4; x++) acc += f[x] * part[x][j][e][lane];
            const int row = 8 * (e >> 2) + 4 * h + (e & 3);          // Oᵀ row of tile j: d = DT·row + j
            o[(long long)(q0 + r) * D + DT * row + j] = acc * inv;
        }
    }
}

#endif
