// anvil_attn_train.h — causal self-attention for training on CDNA4 matrix cores, with neither the
// scores S nor the probabilities P in memory.
//
// For each (batch n, head h) with T queries and keys of D features:
//   S[t][u] = alpha · Σ_c Q[t][c] K[u][c] for u ≤ t (keys past the query are masked out)
//   m[t] = max_u S[t][u],  l[t] = Σ_u exp(S[t][u] − m[t]),  P = exp(S − m) / l,  O = P V
// and, given dO, the gradient
//   dP = dO Vᵀ,  Drow[t] = Σ_c dO[t][c] O[t][c] (= Σ_u dP[t][u] P[t][u]),  dS = P ⊙ (dP − Drow)
//   dQ = alpha · dS K,  dK = alpha · dSᵀ Q,  dV = Pᵀ dO
// (what the front end's softmax(q kᵀ · alpha − C · (u > t)) v and its adjoint compute for a mask
// constant C large enough that exp of a masked score is exactly 0 in float32, with the sums taken
// in another order). Key tiles past a query tile's diagonal are skipped; on the diagonal tile the
// masked scores are −inf (forward) or their P is 0 (backward). Scores are kept in base 2: the Q (or
// K) operand is scaled by alpha · log2(e), so P = 2^(S₂ − m₂) / l on v_exp_f32, and m holds m₂.
//
// Work is cut in 32-row tiles (NT = T / 32 per head). A workgroup takes the pair of tiles p and
// NT − 1 − p of one head, which together meet NT + 1 (query tile, key tile) pairs under the causal
// mask whatever p is, so every workgroup has the same work. Its eight wavefronts are (tile of the
// pair, split s = 0..3): the tiles of the other side are staged in LDS four at a time (one per s),
// shared by both tiles of the pair, and wavefront (i, s) takes the staged tile s of each round. The
// four splits of a tile are combined through LDS in split order (deterministic) at the end.
//
// fp32 MFMA 32x32x2: lane l (r = l % 32, half h = l / 32) gives A[r][h] and B[h][r] and holds
// C[8(e/4) + 4h + e%4][r] in accumulator e. Products whose k runs over features use the row form of
// both operands (lane r's row, features D/2·h .. D/2·h + D/2 − 1); products whose k runs over the
// rows of a tile take the accumulator just computed as B (its element e is k-slot h of MFMA e) and
// the other operand in column form (row 8(e/4) + 4h + e%4, feature D/32·r + j for output tile j).
//
// Three launches: the forward writes O and the row statistics m₂ and l; the backward's dQ launch
// (query tiles, K and V staged; it also writes Drow) and dK/dV launch (key tiles: their own K and V
// rows in LDS, Q, dO and the row statistics staged) each recompute P from Q, K, m₂ and l.
#pragma once
#ifndef ANVIL_EMULATE

struct anvil_attn_io {
    const float *q, *k, *v;          // Q, K, V: element (n, h, t, c) at n·qn + h·qh + t·qs + c
    long long qn, qh, qs;
    float *o;                        // O (written by the forward, read by the backward) and dO:
    const float *dout;               //   element (n, h, t, c) at n·on + h·oh + t·os + c
    long long on, oh, os;
    float *m, *l;                    // row statistics: element (n, h, t) at (n·H + h)·T + t
    float *drow;                     // Drow, in the row statistics' layout (dQ launch → dK/dV launch)
    float *dq, *dk, *dv;             // gradients, in Q's layout
    int H, BH;                       // heads, and batch × heads
    float alpha;
};

// LDS row pitch of a staged 32 x D tile: D + 4 floats keeps the row-form reads (32 rows, one
// 16-byte column each) on distinct banks
template <int D, int TI, int SL = 4> struct anvil_at_shape {
    static constexpr int P = D + 4;
    static constexpr int DH = D / 2, DT = D / 32;
    static constexpr int TILE = 32 * P;
    // forward and dQ: K and V tiles; dK/dV: Q and dO tiles plus m, l, Drow
    static constexpr int STAGE = SL * (2 * TILE + 96);
    // partial output tiles of the 4·TI wavefronts, one accumulator register (64 lanes) per LDS row of
    // 65 words: written lane by lane, and read one output row at a time (64 features on 64 lanes,
    // drawn from two lanes' registers e = 0..15 of DT tiles) without two lanes meeting on a bank
    static constexpr int PART = TI * 4 * DT * 16 * 65;
    static constexpr int WORDS = STAGE > PART ? STAGE : PART;
};

// Workgroup L of a grid of per · BH: head bh and index x in [0, per). Workgroups go to the 8 XCDs
// round-robin by id; when BH is a multiple of 8 all workgroups of one head land on one XCD, whose L2
// then holds that head's Q, K, V (and dO, O).
__device__ __forceinline__ void anvil_at_place(int L, int per, int BH, int &bh, int &x) {
    if (BH % 8 == 0) {
        const int xcd = L & 7, idx = L >> 3;
        bh = 8 * (idx / per) + xcd;
        x = idx % per;
    } else {
        bh = L / per;
        x = L % per;
    }
}

// workgroups per head: one per tile, or one per pair of tiles p, NT − 1 − p
__host__ __device__ constexpr int anvil_at_groups(int NT, int TI) { return TI == 2 ? (NT + 1) / 2 : NT; }

// tiles of the other side staged at once by the forward and dQ: all of them when a pair's 8 fit
// in LDS (T ≤ 256: one round, no barrier between a wavefront's tiles), else rounds of 4
__host__ __device__ constexpr int anvil_at_slots(int NT, int TI) { return TI == 2 && NT > 4 && NT <= 8 ? 8 : 4; }

template <int D>
__device__ __forceinline__ float anvil_at_comp(const typename anvil_vec_of<D>::type &x, int j) {
    if constexpr (D == 32) return x;
    else return x[j];
}

// Sum of the four splits' partial tiles for tile ti of the pair (rows of the tile, features d) into
// dst (row stride ds), scaled by f[x][row] / div[row] where given; wavefront s stores rows 8s .. 8s+7.
template <int D, bool ACC>
__device__ __forceinline__ void anvil_at_store(const float *part, int ti, int s, int lane, float *dst,
                                               long long ds, const float *fx, const float *div, float scale) {
    constexpr int DT = D / 32;
    for (int rr = 0; rr < 8; rr++) {
        const int row = 8 * s + rr;
        float f[4] = {1.f, 1.f, 1.f, 1.f};
        float g = scale;
        if (fx) {
#pragma unroll
            for (int x = 0; x < 4; x++) f[x] = fx[x * 32 + row];
            g = scale / div[row];
        }
        for (int d = lane; d < D; d += 64) {
            const int j = d % DT, i = d / DT;
            const int e = 4 * (i >> 3) + (i & 3), src = row + 32 * ((i >> 2) & 1);
            float acc = 0.f;
#pragma unroll
            for (int x = 0; x < 4; x++) acc += part[(((ti * 4 + x) * DT + j) * 16 + e) * 65 + src] * f[x];
            float *p = dst + (long long)row * ds + d;
            *p = ACC ? *p + acc * g : acc * g;
        }
    }
}

// The K and V tiles 4·rd .. 4·rd + 3 (those ≤ last) of one head, in two steps: the lane's share of
// them loaded into registers (all loads issued together), then stored to LDS. The loads of round
// rd + 1 are issued before round rd's products, so they are in flight while those run.
template <int D, int TI, int SL> struct anvil_at_kv { anvil_f32x4 x[SL * 2 * 32 * (D / 4) / (256 * TI)]; };

template <int D, int TI, int SL>
__device__ __forceinline__ void anvil_at_load_kv(anvil_at_kv<D, TI, SL> &b, const float *kb, const float *vb,
                                                 long long qs, int rd, int last) {
    constexpr int C4 = D / 4, PER = SL * 2 * 32 * C4 / (256 * TI);
#pragma unroll
    for (int it = 0; it < PER; it++) {
        const int i = threadIdx.x + 256 * TI * it;
        const int c4 = i % C4, row = (i / C4) % 32, which = (i / (32 * C4)) & 1, j = i / (64 * C4);
        const int kt = SL * rd + j;
        if (kt <= last) b.x[it] = *(const anvil_f32x4 *)((which ? vb : kb) + (long long)(32 * kt + row) * qs + 4 * c4);
    }
}

template <int D, int TI, int SL>
__device__ __forceinline__ void anvil_at_put_kv(float *lds, const anvil_at_kv<D, TI, SL> &b, int rd, int last) {
    typedef anvil_at_shape<D, TI, SL> S;
    constexpr int C4 = D / 4, PER = SL * 2 * 32 * C4 / (256 * TI);
#pragma unroll
    for (int it = 0; it < PER; it++) {
        const int i = threadIdx.x + 256 * TI * it;
        const int c4 = i % C4, row = (i / C4) % 32, which = (i / (32 * C4)) & 1, j = i / (64 * C4);
        if (SL * rd + j <= last) *(anvil_f32x4 *)&lds[(2 * j + which) * S::TILE + row * S::P + 4 * c4] = b.x[it];
    }
}

// ------------------------------------------------------------------------------------------ forward
// grid: anvil_at_groups<NT, TI> · BH workgroups of 256·TI lanes
template <int D, int NT, int TI>
__device__ __forceinline__ void anvil_attn_fwd(const anvil_attn_io &a) {
    constexpr int SL = anvil_at_slots(NT, TI);
    typedef anvil_at_shape<D, TI, SL> S;
    constexpr int DH = S::DH, DT = S::DT, P = S::P;
    typedef typename anvil_vec_of<D>::type vec;
    __shared__ float lds[S::WORDS];
    __shared__ float stat[TI][2][4][32];               // [tile][m, l][split][row]
    __shared__ float fac[TI][4][32], tot[TI][32];
    int bh, p;
    anvil_at_place(blockIdx.x, anvil_at_groups(NT, TI), a.BH, bh, p);
    const int n = bh / a.H, hh = bh - n * a.H;
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ti = w >> 2, s = w & 3;
    const int qt = ti ? NT - 1 - p : p;
    const bool live = !(ti && qt == p);                  // the middle tile of an odd NT is tile 0's
    const int query = 32 * qt + r;
    const float *qb = a.q + n * a.qn + hh * a.qh, *kb = a.k + n * a.qn + hh * a.qh, *vb = a.v + n * a.qn + hh * a.qh;
    // the query row, scaled by alpha · log2(e): scores come out in base 2 (p = 2^(s - m))
    const float sc = a.alpha * 1.4426950408889634f;
    anvil_f32x4 qr[DH / 4];
#pragma unroll
    for (int c = 0; c < DH / 4; c++) qr[c] = sc * *(const anvil_f32x4 *)(qb + (long long)query * a.qs + DH * h + 4 * c);
    anvil_f32x16 oacc[DT];
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[j][e] = 0.f;
    float mrun = -__builtin_inff(), lrun = 0.f;
    const int last = TI == 2 ? NT - 1 - p : p;           // the last key tile the workgroup needs
    anvil_at_kv<D, TI, SL> buf;
    anvil_at_load_kv<D, TI, SL>(buf, kb, vb, a.qs, 0, last);
    for (int rd = 0; rd <= last / SL; rd++) {
        if (rd) __syncthreads();
        anvil_at_put_kv<D, TI, SL>(lds, buf, rd, last);
        __syncthreads();
        if (rd + 1 <= last / SL) anvil_at_load_kv<D, TI, SL>(buf, kb, vb, a.qs, rd + 1, last);
        // the wavefront's staged tiles of the round, back to back: slots s, s + 4, ...
#pragma unroll
        for (int u = 0; u < SL / 4; u++) {
            const int slot = s + 4 * u, kt = SL * rd + slot;
            if (!live || kt > qt) continue;
            const float *ks = lds + (2 * slot) * S::TILE, *vs = lds + (2 * slot + 1) * S::TILE;
            anvil_f32x16 st;
#pragma unroll
            for (int e = 0; e < 16; e++) st[e] = 0.f;
#pragma unroll
            for (int c = 0; c < DH / 4; c++) {
                const anvil_f32x4 kx = *(const anvil_f32x4 *)&ks[r * P + DH * h + 4 * c];
#pragma unroll
                for (int x = 0; x < 4; x++) st = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[x], qr[c][x], st, 0, 0, 0);
            }
            // the V operands of P·V, read now: their LDS latency passes under the softmax
            vec vx[16];
#pragma unroll
            for (int e = 0; e < 16; e++) vx[e] = *(const vec *)&vs[(8 * (e >> 2) + 4 * h + (e & 3)) * P + DT * r];
            __builtin_amdgcn_sched_barrier(0);
            if (kt == qt) {                                 // the diagonal tile: keys past the query
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (8 * (e >> 2) + 4 * h + (e & 3) > r) st[e] = -__builtin_inff();
            }
            float mx = st[0];
#pragma unroll
            for (int e = 1; e < 16; e++) mx = fmaxf(mx, st[e]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));        // finite: key 32·kt ≤ the query
            const float mnew = fmaxf(mrun, mx);
            float ps = 0.f;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                st[e] = __builtin_amdgcn_exp2f(st[e] - mnew);
                ps += st[e];
            }
            ps += __shfl_xor(ps, 32, 64);
            if (kt >= 4) {                                  // not the wavefront's first tile: rescale
                const float corr = __builtin_amdgcn_exp2f(mrun - mnew);
                lrun = lrun * corr + ps;
#pragma unroll
                for (int j = 0; j < DT; j++)
#pragma unroll
                    for (int e = 0; e < 16; e++) oacc[j][e] *= corr;
            } else {
                lrun = ps;
            }
            mrun = mnew;
#pragma unroll
            for (int e = 0; e < 16; e++)
#pragma unroll
                for (int j = 0; j < DT; j++)
                    oacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(anvil_at_comp<D>(vx[e], j), st[e], oacc[j], 0, 0, 0);
        }
    }
    __syncthreads();                                     // staged tiles read: LDS becomes partials
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) lds[(((ti * 4 + s) * DT + j) * 16 + e) * 65 + lane] = oacc[j][e];
    if (h == 0) {
        stat[ti][0][s][r] = mrun;
        stat[ti][1][s][r] = lrun;
    }
    __syncthreads();
    if (s == 0 && h == 0) {                              // per row: the max, each split's factor, l
        float M = stat[ti][0][0][r];
#pragma unroll
        for (int x = 1; x < 4; x++) M = fmaxf(M, stat[ti][0][x][r]);
        float L = 0.f;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const float f = __builtin_amdgcn_exp2f(stat[ti][0][x][r] - M);   // 0 for a split with no tile
            fac[ti][x][r] = f;
            L += stat[ti][1][x][r] * f;
        }
        tot[ti][r] = L;
        if (live) {
            const long long row = (long long)bh * (32 * NT) + query;
            a.m[row] = M;
            a.l[row] = L;
        }
    }
    __syncthreads();
    if (live)
        anvil_at_store<D, false>(lds, ti, s, lane, a.o + n * a.on + hh * a.oh + (long long)(32 * qt) * a.os, a.os,
                                 &fac[ti][0][0], tot[ti], 1.f);
}

// ----------------------------------------------------------------------------------------- backward
// dQ for the query tiles p and NT − 1 − p of head bh
// grid: anvil_at_groups<NT, TI> · BH workgroups of 256·TI lanes
template <int D, int NT, int TI, bool ACC>
__device__ __forceinline__ void anvil_attn_bwd_q_body(const anvil_attn_io &a, float *lds, int bh, int p) {
    constexpr int SL = anvil_at_slots(NT, TI);
    typedef anvil_at_shape<D, TI, SL> S;
    constexpr int DH = S::DH, DT = S::DT, P = S::P;
    typedef typename anvil_vec_of<D>::type vec;
    const int n = bh / a.H, hh = bh - n * a.H;
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ti = w >> 2, s = w & 3;
    const int qt = ti ? NT - 1 - p : p;
    const bool live = !(ti && qt == p);
    const int query = 32 * qt + r;
    const long long qoff = n * a.qn + hh * a.qh, ooff = n * a.on + hh * a.oh;
    const float *kb = a.k + qoff, *vb = a.v + qoff;
    anvil_f32x4 qr[DH / 4], dr[DH / 4];
    float drow = 0.f;
    {
        const float *qp = a.q + qoff + (long long)query * a.qs + DH * h;
        const float *dp = a.dout + ooff + (long long)query * a.os + DH * h;
        const float *op = a.o + ooff + (long long)query * a.os + DH * h;
        const float sc = a.alpha * 1.4426950408889634f;     // scores in base 2, as the forward's
#pragma unroll
        for (int c = 0; c < DH / 4; c++) {
            qr[c] = sc * *(const anvil_f32x4 *)(qp + 4 * c);
            dr[c] = *(const anvil_f32x4 *)(dp + 4 * c);
            const anvil_f32x4 ox = *(const anvil_f32x4 *)(op + 4 * c);
            drow += dr[c].x * ox.x + dr[c].y * ox.y + dr[c].z * ox.z + dr[c].w * ox.w;
        }
        drow += __shfl_xor(drow, 32, 64);
    }
    const long long srow = (long long)bh * (32 * NT) + query;
    const float mq = a.m[srow], rl = 1.f / a.l[srow];
    if (a.drow && live && s == 0 && h == 0) a.drow[srow] = drow;    // for a dK/dV launch that follows
    anvil_f32x16 qacc[DT];
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) qacc[j][e] = 0.f;
    const int last = TI == 2 ? NT - 1 - p : p;
    // eight tiles (one round) are staged in two halves of four: the registers of the whole round
    // would not fit beside the query's Q and dO rows
    constexpr bool halves = SL == 8;
    anvil_at_kv<D, TI, halves ? 4 : SL> buf;
    if constexpr (!halves) anvil_at_load_kv<D, TI, SL>(buf, kb, vb, a.qs, 0, last);
    for (int rd = 0; rd <= last / SL; rd++) {
        if (rd) __syncthreads();
        if constexpr (halves) {
            anvil_at_load_kv<D, TI, 4>(buf, kb, vb, a.qs, 0, last);
            anvil_at_put_kv<D, TI, 4>(lds, buf, 0, last);
            anvil_at_load_kv<D, TI, 4>(buf, kb, vb, a.qs, 1, last);
            anvil_at_put_kv<D, TI, 4>(lds + 8 * S::TILE, buf, 1, last);
        } else {
            anvil_at_put_kv<D, TI, SL>(lds, buf, rd, last);
        }
        __syncthreads();
        if constexpr (!halves) {
            if (rd + 1 <= last / SL) anvil_at_load_kv<D, TI, SL>(buf, kb, vb, a.qs, rd + 1, last);
        }
        // the wavefront's staged tiles of the round, back to back: slots s, s + 4, ...
#pragma unroll
        for (int u = 0; u < SL / 4; u++) {
            const int slot = s + 4 * u, kt = SL * rd + slot;
            if (!live || kt > qt) continue;
            const float *ks = lds + (2 * slot) * S::TILE, *vs = lds + (2 * slot + 1) * S::TILE;
            anvil_f32x16 st, dpt;
#pragma unroll
            for (int e = 0; e < 16; e++) st[e] = dpt[e] = 0.f;
#pragma unroll
            for (int c = 0; c < DH / 4; c++) {
                const anvil_f32x4 kx = *(const anvil_f32x4 *)&ks[r * P + DH * h + 4 * c];
                const anvil_f32x4 vx = *(const anvil_f32x4 *)&vs[r * P + DH * h + 4 * c];
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[x], qr[c][x], st, 0, 0, 0);
                    dpt = __builtin_amdgcn_mfma_f32_32x32x2f32(vx[x], dr[c][x], dpt, 0, 0, 0);
                }
            }
            // the K operands of dS·K, read now: their LDS latency passes under P and dS
            vec kc[16];
#pragma unroll
            for (int e = 0; e < 16; e++) kc[e] = *(const vec *)&ks[(8 * (e >> 2) + 4 * h + (e & 3)) * P + DT * r];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float pe = __builtin_amdgcn_exp2f(st[e] - mq) * rl;
                st[e] = pe * (dpt[e] - drow);                // dSᵀ
            }
            if (kt == qt) {                                 // the diagonal tile: keys past the query
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (8 * (e >> 2) + 4 * h + (e & 3) > r) st[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 16; e++)
#pragma unroll
                for (int j = 0; j < DT; j++)
                    qacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(anvil_at_comp<D>(kc[e], j), st[e], qacc[j], 0, 0, 0);
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) lds[(((ti * 4 + s) * DT + j) * 16 + e) * 65 + lane] = qacc[j][e];
    __syncthreads();
    if (live)
        anvil_at_store<D, ACC>(lds, ti, s, lane, a.dq + qoff + (long long)(32 * qt) * a.qs, a.qs, nullptr, nullptr,
                               a.alpha);
}

// dK and dV for the key tiles p and NT − 1 − p of head bh
// grid: anvil_at_groups<NT, TI> · BH workgroups of 256·TI lanes
// OWN: Drow computed here from dO and O while staging (when no dQ launch precedes this one)
template <int D, int NT, int TI, bool ACC, bool OWN>
__device__ __forceinline__ void anvil_attn_bwd_kv_body(const anvil_attn_io &a, float *lds, int bh, int p) {
    typedef anvil_at_shape<D, TI> S;
    constexpr int DH = S::DH, DT = S::DT, P = S::P, C4 = D / 4;
    typedef typename anvil_vec_of<D>::type vec;
    float (*kvs)[2][S::TILE] = (float (*)[2][S::TILE])(lds + S::WORDS);     // the workgroup's key tiles: K (scaled), V
    const int n = bh / a.H, hh = bh - n * a.H;
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ti = w >> 2, s = w & 3;
    const int kt = ti ? NT - 1 - p : p;
    const bool live = !(ti && kt == p);
    const long long qoff = n * a.qn + hh * a.qh, ooff = n * a.on + hh * a.oh;
    const float *qb = a.q + qoff, *db = a.dout + ooff, *ob = a.o + ooff;
    const long long sb = (long long)bh * (32 * NT);
    const float *mb = a.m + sb, *lb = a.l + sb, *rb = OWN ? nullptr : a.drow + sb;
    {
        // the K and V rows of the workgroup's key tiles, K scaled by alpha · log2(e) (scores in base
        // 2, as the forward's); visible after the first round's barrier
        const float sc = a.alpha * 1.4426950408889634f;
        constexpr int ITEMS = TI * 2 * 32 * C4, PK = (ITEMS + 256 * TI - 1) / (256 * TI);
        anvil_f32x4 x[PK];
#pragma unroll
        for (int it = 0; it < PK; it++) {
            const int i = threadIdx.x + 256 * TI * it;
            const int c4 = i % C4, row = (i / C4) % 32, which = (i / (32 * C4)) & 1, t2 = i / (64 * C4);
            const int kt2 = t2 ? NT - 1 - p : p;
            if (i < ITEMS)
                x[it] = *(const anvil_f32x4 *)((which ? a.v : a.k) + qoff + (long long)(32 * kt2 + row) * a.qs + 4 * c4);
        }
#pragma unroll
        for (int it = 0; it < PK; it++) {
            const int i = threadIdx.x + 256 * TI * it;
            const int c4 = i % C4, row = (i / C4) % 32, which = (i / (32 * C4)) & 1, t2 = i / (64 * C4);
            if (i < ITEMS) *(anvil_f32x4 *)&kvs[t2][which][row * P + 4 * c4] = which ? x[it] : sc * x[it];
        }
    }
    const float *kr = kvs[ti][0], *vr = kvs[ti][1];
    anvil_f32x16 kacc[DT], vacc[DT];
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) kacc[j][e] = vacc[j][e] = 0.f;
    // staged query tile j of a round: Q at j·(2·TILE + 96), dO one TILE later, then m, 1 / l, Drow
    constexpr int PER = 4 * 32 * C4 / (256 * TI);
    for (int rd = 0; p + 4 * rd < NT; rd++) {
        if (rd) __syncthreads();
        // every load of the round, then the LDS stores (one wait for memory per round)
        anvil_f32x4 qx[PER], dx[PER], ox[OWN ? PER : 1];
        float sx[PER];
#pragma unroll
        for (int it = 0; it < PER; it++) {
            const int i = threadIdx.x + 256 * TI * it;
            const int c4 = i % C4, row = (i / C4) % 32, j = i / (32 * C4);
            const int qt = p + 4 * rd + j;
            if (qt < NT) {
                const long long t = 32 * qt + row;
                qx[it] = *(const anvil_f32x4 *)(qb + t * a.qs + 4 * c4);
                dx[it] = *(const anvil_f32x4 *)(db + t * a.os + 4 * c4);
                if constexpr (OWN) ox[it] = *(const anvil_f32x4 *)(ob + t * a.os + 4 * c4);
                if (c4 < (OWN ? 2 : 3)) sx[it] = (c4 == 0 ? mb : c4 == 1 ? lb : rb)[t];
            }
        }
#pragma unroll
        for (int it = 0; it < PER; it++) {
            const int i = threadIdx.x + 256 * TI * it;
            const int c4 = i % C4, row = (i / C4) % 32, j = i / (32 * C4);
            const int qt = p + 4 * rd + j;
            float *base = lds + j * (2 * S::TILE + 96);
            if (qt < NT) {
                *(anvil_f32x4 *)&base[row * P + 4 * c4] = qx[it];
                *(anvil_f32x4 *)&base[S::TILE + row * P + 4 * c4] = dx[it];
                if (c4 < (OWN ? 2 : 3)) base[2 * S::TILE + 32 * c4 + row] = c4 == 1 ? 1.f / sx[it] : sx[it];
            }
            if constexpr (OWN) {
                // Drow of the row: its C4 lanes' partial dot products, added across them
                float part = qt < NT ? dx[it].x * ox[it].x + dx[it].y * ox[it].y + dx[it].z * ox[it].z +
                                           dx[it].w * ox[it].w : 0.f;
#pragma unroll
                for (int x = 1; x < C4; x <<= 1) part += __shfl_xor(part, x, 64);
                if (qt < NT && c4 == 0) base[2 * S::TILE + 64 + row] = part;
            }
        }
        __syncthreads();
        const int qt = p + 4 * rd + s;
        if (live && qt < NT && qt >= kt) {
            const float *base = lds + s * (2 * S::TILE + 96);
            const float *qs_ = base, *ds_ = base + S::TILE, *ms = base + 2 * S::TILE;
            anvil_f32x16 st, dpt;
#pragma unroll
            for (int e = 0; e < 16; e++) st[e] = dpt[e] = 0.f;
#pragma unroll
            for (int c = 0; c < DH / 4; c++) {
                const anvil_f32x4 qx = *(const anvil_f32x4 *)&qs_[r * P + DH * h + 4 * c];
                const anvil_f32x4 dx = *(const anvil_f32x4 *)&ds_[r * P + DH * h + 4 * c];
                const anvil_f32x4 kx = *(const anvil_f32x4 *)&kr[r * P + DH * h + 4 * c];
                const anvil_f32x4 vx = *(const anvil_f32x4 *)&vr[r * P + DH * h + 4 * c];
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(qx[x], kx[x], st, 0, 0, 0);
                    dpt = __builtin_amdgcn_mfma_f32_32x32x2f32(dx[x], vx[x], dpt, 0, 0, 0);
                }
            }
            // st[e], dpt[e]: S and dP at query row 8(e/4) + 4h + e%4 of tile qt, key r of tile kt
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = 8 * (e >> 2) + 4 * h + (e & 3);
                const float pe = __builtin_amdgcn_exp2f(st[e] - ms[row]) * ms[32 + row];
                st[e] = pe;
                dpt[e] = pe * (dpt[e] - ms[64 + row]);       // dS
            }
            if (kt == qt) {                                 // the diagonal tile: queries before the key
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (r > 8 * (e >> 2) + 4 * h + (e & 3)) st[e] = dpt[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = 8 * (e >> 2) + 4 * h + (e & 3);
                const vec dx = *(const vec *)&ds_[row * P + DT * r];
                const vec qx = *(const vec *)&qs_[row * P + DT * r];
#pragma unroll
                for (int j = 0; j < DT; j++) {
                    vacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(anvil_at_comp<D>(dx, j), st[e], vacc[j], 0, 0, 0);
                    kacc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(anvil_at_comp<D>(qx, j), dpt[e], kacc[j], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) lds[(((ti * 4 + s) * DT + j) * 16 + e) * 65 + lane] = vacc[j][e];
    __syncthreads();
    if (live)
        anvil_at_store<D, ACC>(lds, ti, s, lane, a.dv + qoff + (long long)(32 * kt) * a.qs, a.qs, nullptr, nullptr, 1.f);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) lds[(((ti * 4 + s) * DT + j) * 16 + e) * 65 + lane] = kacc[j][e];
    __syncthreads();
    if (live)
        anvil_at_store<D, ACC>(lds, ti, s, lane, a.dk + qoff + (long long)(32 * kt) * a.qs, a.qs, nullptr, nullptr,
                               a.alpha);
}

// The backward as two launches: dQ (writes Drow), then dK/dV.
// grid: anvil_at_groups<NT, TI> · BH workgroups of 256·TI lanes each
template <int D, int NT, int TI, bool ACC>
__device__ __forceinline__ void anvil_attn_bwd_q(const anvil_attn_io &a) {
    __shared__ float lds[anvil_at_shape<D, TI, anvil_at_slots(NT, TI)>::WORDS];
    int bh, p;
    anvil_at_place(blockIdx.x, anvil_at_groups(NT, TI), a.BH, bh, p);
    anvil_attn_bwd_q_body<D, NT, TI, ACC>(a, lds, bh, p);
}

template <int D, int NT, int TI, bool ACC>
__device__ __forceinline__ void anvil_attn_bwd_kv(const anvil_attn_io &a) {
    typedef anvil_at_shape<D, TI> S;
    __shared__ float lds[S::WORDS + TI * 2 * S::TILE];
    int bh, p;
    anvil_at_place(blockIdx.x, anvil_at_groups(NT, TI), a.BH, bh, p);
    anvil_attn_bwd_kv_body<D, NT, TI, ACC, false>(a, lds, bh, p);
}

// The backward as one launch whose workgroups alternate between the two (dK/dV computing Drow
// itself): for short heads, where the launches are mostly fixed cost and running the two side by
// side halves it. grid: 2 · anvil_at_groups<NT, TI> · BH workgroups of 256·TI lanes.
template <int D, int NT, int TI, bool ACC>
__device__ __forceinline__ void anvil_attn_bwd(const anvil_attn_io &a) {
    typedef anvil_at_shape<D, TI, anvil_at_slots(NT, TI)> SQ;
    typedef anvil_at_shape<D, TI> SK;
    constexpr int WQ = SQ::WORDS, WK = SK::WORDS + TI * 2 * SK::TILE;
    __shared__ float lds[WQ > WK ? WQ : WK];
    int bh, x;
    anvil_at_place(blockIdx.x, 2 * anvil_at_groups(NT, TI), a.BH, bh, x);
    if (x & 1) anvil_attn_bwd_kv_body<D, NT, TI, ACC, true>(a, lds, bh, x >> 1);
    else anvil_attn_bwd_q_body<D, NT, TI, ACC>(a, lds, bh, x >> 1);
}

#endif
