// gdn_prefill.hip — chunked (WY/UT) prefill of T tokens of one sequence.
//
// Same recurrence as the decode path (overhang engines/qwen.c:307-358, one
// token at a time there), evaluated chunk-wise as transformers'
// torch_chunk_gated_delta_rule does (modeling_qwen3_5_moe.py:250-328):
// for a chunk of C = 64 tokens with cumulative log-decay gc,
//     L  = strict_lower(beta_i k_i.k_j exp(gc_i - gc_j)),   X = (I + L)^-1
//     W  = X (K * beta * e^gc),   U = X (V * beta)
//     Aqk = lower_incl_diag(q_i.k_j exp(gc_i - gc_j))
//     v_new = U - W S;   o = (Q * e^gc) S + Aqk v_new   (S = the chunk's starting state)
//     S <- e^{gc_last} S + (K * e^{gc_last - gc})^T v_new
// Only exp of differences of cumulative decays are formed, never exp(-gc).
//
// Three launches, all on the caller's stream:
//   P1 wy      per (key head, chunk) with its value heads: conv + SiLU, q/k
//              L2 norm, gates, KK^T, QK^T, (I+L)^-1 blocks, W, U on fp32
//              MFMA, written as per-lane fragment panels           MFMA-bound
//   P3 scan    per (value head, 16-column block of S): the chunk
//              recurrence and the raw outputs, sequential over chunks, on
//              fp32 MFMA                                           MFMA-bound
//   P4 norm    gated RMSNorm of the head outputs                   HBM-bound
//              + P2 commit (extra blocks of the same launch): conv history
//              ring -> last K-1 inputs, new phase                  tiny
//
// MFMA conventions (v_mfma_f32_16x16x4_f32, lane l, g = l / 16):
//   A[16][4]: lane holds A[l%16][g];  B[4][16]: lane holds B[g][l%16];
//   D[16][16]: lane holds D[4g + r][l%16] in register r.
// A tile held in D layout can feed the B operand of the next product: at
// k-step s, lane group g supplies row 4g+s of the tile (its register s);
// the matching A fragment is read with the same permuted k index.  P3 keeps
// S and v_new in registers this way for the whole scan.
#include "omh_device.h"
#include "omh_internal.h"
#include <type_traits>

namespace omh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int C = kChunk;

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f v4zero() { v4f z = {0.f, 0.f, 0.f, 0.f}; return z; }

// Scan work split for head dim D: eight waves per workgroup, which owns a
// D x 16 column slice of S; wave w < NST = D/16 holds row tile w (16 kd
// rows) in registers.  Per chunk, waves 0-3 form v_new of token tile w
// (W S over all of kd) and waves 4-7 the output of token tile w - 4.
// Panels, per lane, in MFMA fragment order (the WY kernel writes them):
//   W           per (value head, chunk, token tile j): f = kt*4 + s -> row 16j + l%16, col 16kt + 4g + s
//   q^          per (key head, chunk, token tile j): the same layout
//   k^T         per (key head, chunk, row tile w): f = tt*4 + s -> row 16tt + 4g + s, col 16w + l%16
//   Aqk         per (value head, chunk, token tile mt): f = kt*4 + s -> row 16mt + l%16, col 16kt + 4g + s
//   U           per (value head, chunk, column block cb, mt): f = r -> row 16mt + 4g + r, col 16cb + l%16
// q^ and k^ are the normalised q, k, shared by the value heads of a key
// head; their per-value-head token scalings e^gc and e^{gl-gc} go with them
// as two 64-float vectors per (value head, chunk).
// (g = l / 16); each group of four consecutive f is one float4 per lane.
template <int D>
struct ScanShape {
    static constexpr int NST = D / 16;          // S row tiles
    static constexpr int NWV = 8;
    static_assert(NST >= 1 && NST <= NWV, "scan split");
};
// float4 index of panel group f4 of lane l in block `blk` (4 groups per block)
__device__ __forceinline__ size_t pan4(size_t blk, int f4, int l) { return ((blk * 4 + f4) * OMH_WAVE + l) * 4; }
// W / q^ panels: group kt of token tile j (NST groups per tile)
template <int D>
__device__ __forceinline__ size_t panj(size_t hc, int j, int kt, int l) {
    return (((hc * 4 + j) * (D / 16) + kt) * OMH_WAVE + l) * 4;
}

// ---------------------------------------------------------------- P2 commit
// New conv history = last K-1 entries of [old history, x_0 .. x_{T-1}] for
// phase (p + T) mod ring size.  A token's ring slot is its index mod the
// ring size, so old history values that stay are already in place: only
// the new inputs among the last K-1 are written.  Every block reads the
// phase from phase[epoch]; the new one goes to phase[1 - epoch] (block 0
// also carries the other sequences' phases over) and the host flips the
// layer's epoch after the launch, as for decode launches.  Runs as extra
// 256-thread blocks of the gated-norm launch (after the WY kernel, which
// reads the old history).
__device__ __forceinline__ void conv_commit(const PrefillArgs &a, int conv_dim, int blk) {
    const int c = blk * 256 + threadIdx.x;
    const int K = a.K, T = a.T;
    const int ph = a.L.phase[a.L.epoch * a.L.max_seqs + a.seq];
    const int nph = (ph + T) & (kConvRing - 1);
    if (c < conv_dim) {
        float *rs = a.L.conv_st + ring_at(a.seq, 0, c, conv_dim);
        for (int j = 0; j < K - 1; j++) {
            const int idx = T + j;               // index into [old history (K-1), x_0 ..]
            if (idx >= K - 1)
                rs[(size_t)ring_slot(nph, K, j) * conv_dim] = a.qkv[(size_t)(idx - (K - 1)) * a.ld_qkv + c];
        }
    }
    if (blk == 0) {
        int *nxt = a.L.phase + (1 - a.L.epoch) * a.L.max_seqs;
        const int *cur = a.L.phase + a.L.epoch * a.L.max_seqs;
        for (int s = threadIdx.x; s < a.L.max_seqs; s += 256) nxt[s] = s == a.seq ? nph : cur[s];
    }
}

// ---------------------------------------------------------------- P4 norm
// Blocks nnorm and above: the conv-history commit.
template <int D>
__global__ __launch_bounds__(256)
void prefill_gated_norm_kernel(const PrefillArgs a, int nnorm, int conv_dim) {
    if ((int)blockIdx.x >= nnorm) {
        conv_commit(a, conv_dim, blockIdx.x - nnorm);
        return;
    }
    constexpr int LPR = D / 4;                   // lanes per row
    constexpr int RPB = 256 / LPR;               // rows per block
    const int l4 = threadIdx.x % LPR;
    const size_t row = (size_t)blockIdx.x * RPB + threadIdx.x / LPR;
    const int vh = a.vh;
    if (row >= (size_t)a.T * vh) return;
    const size_t t = row / vh;
    const int h = (int)(row % vh);
    float *op = a.core + t * ((size_t)vh * D) + (size_t)h * D + l4 * 4;
    const float4 o = *reinterpret_cast<const float4 *>(op);
    const float4 zz = *reinterpret_cast<const float4 *>(a.z + t * a.ld_z + (size_t)h * D + l4 * 4);
    const float4 gn = *reinterpret_cast<const float4 *>(a.L.gnorm + l4 * 4);
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = omh_xor_sum_below<LPR>(ss);
    const float rn = 1.f / sqrtf(ss / (float)D + a.eps);   // qwen.c:354-357
    float4 y;
    y.x = o.x * rn * gn.x * omh_silu(zz.x);
    y.y = o.y * rn * gn.y * omh_silu(zz.y);
    y.z = o.z * rn * gn.z * omh_silu(zz.z);
    y.w = o.w * rn * gn.w * omh_silu(zz.w);
    *reinterpret_cast<float4 *>(op) = y;
}

// ---------------------------------------------------------------- P1 WY
// One workgroup per (key head, chunk, group of one or two of its value
// heads): the chunk's conv + SiLU and L2 norms straight from mixed_qkv, the
// gates, then on fp32 MFMA
//   G = K K^T, P = Q K^T (lower 16x16 tiles; shared by the group's value heads),
//   per value head: L = strict_lower(beta_i G e^{gc_i-gc_j}),
//   Aqk = lower_incl(P e^{gc_i-gc_j}), X = (I + L)^-1 (four 16x16 diagonal
//   inverses, then blocked forward substitution), W = X (K beta e^gc),
//   U = X (V beta),
// and the operand panels the scan reads.  Threads exchange data through
// LDS only, so every barrier orders LDS alone: the next item's prefetched
// inputs and this item's panel stores stay in flight across them.
template <int D>
struct WyShape {
    static constexpr int NW = D / 16 < 4 ? 4 : D / 16;   // waves
    static constexpr int NT = NW * OMH_WAVE;
    static constexpr int PD = D + 4, PC = C + 4;         // padded LDS rows
    static constexpr int NCT = D / 16;                   // 16-column tiles of D
    // Qs Ks Vs, Ls Xs As, then gc, beta, beta e^gc for two value heads
    static constexpr size_t LDS = (size_t)(3 * C * PD + 3 * C * PC + 6 * C) * sizeof(float);
};

// conv1d over KK taps (the history oldest..newest, then the input; op
// order as engines/qwen.c:311-319) + SiLU over NS consecutive tokens, the
// outputs replacing the inputs in registers; tokens at or past nvalid are
// zero.  The history h0 h1 h2 is the last three inputs (right-aligned: for
// KK < 4 only the last KK-1 are used), w the taps right-aligned (tap j in
// component 4-KK+j).
template <int KK, int NS>
__device__ __forceinline__ void conv_inplace(float (&x)[NS], float h0, float h1, float h2, float4 w, int nvalid) {
    const float wt[4] = {w.x, w.y, w.z, w.w};
    float h[3] = {h0, h1, h2};
#pragma unroll
    for (int t = 0; t < NS; t++) {
        const float xt = x[t];
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KK - 1; j++) acc += wt[4 - KK + j] * h[4 - KK + j];
        acc += wt[3] * xt;
        h[0] = h[1];
        h[1] = h[2];
        h[2] = xt;
        const float y = omh_silu_fast(acc);
        x[t] = t < nvalid ? y : 0.f;
    }
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>)
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// The lower 16x16 tiles of a 64x64 matrix, in order (0,0) (1,0) (1,1) (2,0) ...
__device__ __forceinline__ void lower_tile(int it, int &i, int &j) {
    i = it < 1 ? 0 : (it < 3 ? 1 : (it < 6 ? 2 : 3));
    j = it - i * (i + 1) / 2;
}

// Work item m -> (key head hk, first value head h0, chunk c) for items of
// vpg value heads each (ngrp groups per key head), XCD-aware: with N items
// and a grid that is a multiple of 8, the items a given XCD processes
// together are consecutive (the groups of one key head, then the next key
// head, for one chunk), so the q/k inputs they share are read once per XCD L2.
__device__ __forceinline__ void wy_item(int m, int N, int kh, int rep, int vpg, int &hk, int &h0, int &c, int &grp) {
    const int ngrp = rep / vpg;
    const int mm = N % 8 == 0 ? (m % 8) * (N / 8) + m / 8 : m;
    grp = mm % ngrp;
    hk = (mm / ngrp) % kh;
    c = mm / (ngrp * kh);
    h0 = hk * rep + grp * vpg;
}

// One work item's conv inputs, held in registers: loaded during the item
// before (load), turned into conv + SiLU outputs in place during that item
// (compute_unit, gates), written to LDS when they are needed (store; the
// second value head's v when its turn comes, store_v1).  Unit u of a thread
// is part u (q, k, v of value head 0, v of value head 1) of one (channel,
// NSEG-token segment) pair, so the second value head's v has registers of
// its own; a unit's history is the three inputs before its segment (for
// the first segment of chunk 0 the channel's ring entry).  Gate wave j
// (NW-1-j) carries the gates of value head j of the item for its token.
template <int D, int KK>
struct WyIn {
    static constexpr int NSEG = 16;
    static constexpr int NT = WyShape<D>::NT;
    static constexpr int NPAIR = D * (C / NSEG);            // (channel, segment) pairs per part
    static_assert(NPAIR <= NT, "one pair per thread and part");
    float x[4][NSEG];     // inputs of the segment, then its conv + SiLU outputs
    float4 hv[4];         // the three inputs before the segment in .x .y .z
    float4 wv[4];
    float ga, gb;         // gate inputs of the gate wave's token; then gc and beta

    __device__ __forceinline__ static int channel(const PrefillArgs &a, int part, int h0, int hk) {
        return part == 0 ? hk * D : (part == 1 ? a.kh * D + hk * D : 2 * a.kh * D + (h0 + part - 2) * D);
    }
    // the thread's pair (uniform segment for D a multiple of the wave size)
    __device__ __forceinline__ static bool pair_of(int tid, int &seg, int &cc) {
        seg = tid / D;
        if (D % OMH_WAVE == 0) seg = __builtin_amdgcn_readfirstlane(seg);
        cc = tid % D;
        return NPAIR == NT || tid < NPAIR;
    }

    // parts U0 .. U1-1 (and the gate inputs on the gate waves if gate)
    template <int U0, int U1>
    __device__ __forceinline__ void load(const PrefillArgs &a, int vpg, int h0, int hk, int c, int tid, int gj, bool gate,
                                         int lane, int ph) {
        const int T = a.T, t0 = c * C;
        const size_t ld = a.ld_qkv;
        int seg, cc;
        const bool has = pair_of(tid, seg, cc);
        const int ts = t0 + seg * NSEG;
#pragma unroll
        for (int u = U0; u < U1; u++) {
            if (!has || u - 2 >= vpg) continue;
            const int ch0 = channel(a, u, h0, hk);
            float h0v, h1v, h2v;
            if (ts >= 3 && ts + NSEG <= T) {
                // rows ts-3 .. ts+NSEG-1, one row pointer stepped down the column
                const float *rp = a.qkv + (size_t)(ts - 3) * ld + ch0;
                h0v = rp[cc]; rp += ld;
                h1v = rp[cc]; rp += ld;
                h2v = rp[cc]; rp += ld;
#pragma unroll
                for (int t = 0; t < NSEG; t++) { x[u][t] = rp[cc]; rp += ld; }
            } else {
                // the last segment (rows past T are clamped; their outputs
                // are zeroed) or the first of the sequence (history: the ring)
                const float *col = a.qkv + ch0 + cc;
#pragma unroll
                for (int t = 0; t < NSEG; t++) x[u][t] = col[(size_t)min(ts + t, T - 1) * ld];
                if (ts == 0) {
                    // the ring's K-1 history slots, oldest first, right-aligned
                    // (this waits for the load: once per sequence)
                    const int conv_dim = (2 * a.kh + a.vh) * D;
                    const float *rs = a.L.conv_st + ring_at(a.seq, 0, ch0 + cc, conv_dim);
                    h0v = KK >= 4 ? rs[(size_t)((ph + 1) & (kConvRing - 1)) * conv_dim] : 0.f;
                    h1v = KK >= 3 ? rs[(size_t)((ph + 2) & (kConvRing - 1)) * conv_dim] : 0.f;
                    h2v = rs[(size_t)((ph + 3) & (kConvRing - 1)) * conv_dim];
                } else {
                    h0v = col[(size_t)min(ts - 3, T - 1) * ld];
                    h1v = col[(size_t)min(ts - 2, T - 1) * ld];
                    h2v = col[(size_t)min(ts - 1, T - 1) * ld];
                }
            }
            hv[u] = make_float4(h0v, h1v, h2v, 0.f);
            wv[u] = *reinterpret_cast<const float4 *>(a.L.conv_w + (size_t)(ch0 + cc) * kConvRing);
        }
        if (gate) {
            const int tt = min(t0 + lane, T - 1);
            ga = a.a[(size_t)tt * a.ld_ab + h0 + gj];
            gb = a.b[(size_t)tt * a.ld_ab + h0 + gj];
        }
    }

    // conv + SiLU of part u in place, branch-free
    template <int U>
    __device__ __forceinline__ void compute_unit(const PrefillArgs &a, int c, int tid) {
        int seg, cc;
        if (!pair_of(tid, seg, cc)) return;
        conv_inplace<KK, NSEG>(x[U], hv[U].x, hv[U].y, hv[U].z, wv[U], a.T - (c * C + seg * NSEG));
    }

    // the gates of value head h (qwen.c:337-338, zero past T) with an
    // inclusive prefix sum of g
    __device__ __forceinline__ void gates(const PrefillArgs &a, int h, int c, int lane) {
        float g = 0.f, be = 0.f;
        if (c * C + lane < a.T) {
            g = -expf(a.L.A_log[h]) * omh_softplus(ga + a.L.dt_bias[h]);
            be = omh_sigmoid(gb);
        }
#pragma unroll
        for (int off = 1; off < OMH_WAVE; off <<= 1) {
            const float y = __shfl_up(g, off, OMH_WAVE);
            if (lane >= off) g += y;
        }
        ga = g;
        gb = be;
    }

    // parts U0 .. U1-1 to their LDS tile (Qs, Ks, Vs; part 3 also to Vs)
    template <int U0, int U1>
    __device__ __forceinline__ void store(int tid, float *Qs, float *Ks, float *Vs) {
        constexpr int PD = WyShape<D>::PD;
        int seg, cc;
        if (!pair_of(tid, seg, cc)) return;
#pragma unroll
        for (int u = U0; u < U1; u++) {
            float *dst = (u == 0 ? Qs : (u == 1 ? Ks : Vs)) + seg * NSEG * PD + cc;
#pragma unroll
            for (int t = 0; t < NSEG; t++) dst[t * PD] = x[u][t];
        }
    }
    // the gates to gt (gc, beta, beta e^gc) and the scan's per-token scales
    // of (value head, chunk) hc
    __device__ __forceinline__ void store_gates(const PrefillArgs &a, size_t hc, int lane, float *gt) {
        const float gl = __shfl(ga, C - 1, OMH_WAVE);
        const float ex = expf(ga), ee = expf(gl - ga);
        gt[lane] = ga;
        gt[C + lane] = gb;
        gt[2 * C + lane] = gb * ex;
        a.pg[hc * C + lane] = ex;
        a.pe[hc * C + lane] = ee;
        if (lane == C - 1) a.glast[hc] = ex;
    }
};

// c + A B for 16x16 tiles: A given as the D layout of A^T (lane holds
// A[l%16][4g + s] in register s, the A operand of k-step s), B in D layout
__device__ __forceinline__ v4f mm16(v4f at, v4f b, v4f c) {
#pragma unroll
    for (int s = 0; s < 4; s++) c = mfma4(at[s], b[s], c);
    return c;
}

// (I + N)^-1 for a strictly lower-triangular 16x16 N: with M = -N (M^16 = 0)
// it is (I + M)(I + M^2)(I + M^4)(I + M^8), eight 16x16x16 products on the
// matrix cores.  nd: N in D layout; nt: N^T in D layout.  Returns the
// inverse's transpose in D layout.
__device__ __forceinline__ v4f inv_unit_lower16(v4f nd, v4f nt, int lane) {
    const int l16 = lane % 16, g4 = lane / 16;
    v4f eye;
#pragma unroll
    for (int r = 0; r < 4; r++) eye[r] = 4 * g4 + r == l16 ? 1.f : 0.f;
    const v4f md = -nd, mt = -nt;
    const v4f z = v4zero();
    const v4f m2d = mm16(mt, md, z), m2t = mm16(md, mt, z);
    const v4f m3t = mm16(m2d, mt, z);                       // (M^3)^T = (M^2)^T M^T
    const v4f m4d = mm16(m2t, m2d, z), m4t = mm16(m2d, m2t, z);
    const v4f m8d = mm16(m4t, m4d, z);
    const v4f p1t = eye + mt + m2t + m3t;                   // (I + M + M^2 + M^3)^T
    const v4f p2t = mm16(m4d, p1t, p1t);                    // (P1 + P1 M^4)^T
    return mm16(m8d, p2t, p2t);                             // (P2 + P2 M^8)^T
}

template <int D, int KK>
__global__ __launch_bounds__(WyShape<D>::NT)
void prefill_wy_kernel(const PrefillArgs a) {
    using WS = WyShape<D>;
    using In = WyIn<D, KK>;
    constexpr int NW = WS::NW, PD = WS::PD, PC = WS::PC, NCT = WS::NCT;
    constexpr int NST = ScanShape<D>::NST;

    const int kh = a.kh, rep = a.vh / kh, nc = a.nc;
    const int vpg = rep % 2 == 0 ? 2 : 1;                // value heads per item
    const int nitems = kh * (rep / vpg) * nc;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, g4 = lane / 16;
    const int gj = NW - 1 - wave;                        // value head whose gates this wave carries
    const bool gate = gj < vpg;

    extern __shared__ float smem[];
    float *Qs = smem;                            // [C][PD] q~ -> q^; W staging in the substitution
    float *Ks = Qs + C * PD;                     // [C][PD]
    float *Vs = Ks + C * PD;                     // [C][PD] v of value head 0, then 1
    float *Ls = Vs + C * PD;                     // [C][PC] L
    float *Xs = Ls + C * PC;                     // [C][PC] diagonal blocks of (I + L)^-1
    float *As = Xs + C * PC;                     // [C][PC] Aqk
    float *gts = As + C * PC;                    // [2][3][C] gc, beta, beta e^gc per value head

    // the tiles above the diagonal of L and Aqk stay zero for every item
    for (int e = tid; e < C * C; e += WS::NT) {
        const int row = e / C, col = e % C;
        if (col / 16 > row / 16) { Ls[row * PC + col] = 0.f; As[row * PC + col] = 0.f; }
    }

    const int ph = a.L.phase[a.L.epoch * a.L.max_seqs + a.seq];   // ring phase of the sequence
    int m = blockIdx.x;
    In in;
    if (m < nitems) {
        int hk, h0, c, grp;
        wy_item(m, nitems, kh, rep, vpg, hk, h0, c, grp);
        in.template load<0, 4>(a, vpg, h0, hk, c, tid, gj, gate, lane, ph);
        in.template compute_unit<0>(a, c, tid);
        in.template compute_unit<1>(a, c, tid);
        in.template compute_unit<2>(a, c, tid);
        if (vpg == 2) in.template compute_unit<3>(a, c, tid);
        if (gate) in.gates(a, h0 + gj, c, lane);
    }

    // G and P tiles of this wave (raw, for every value head of the item):
    // G tiles w, w + NW, ..., P tiles (w + 2) mod NW, ...; five products per SIMD
    constexpr int R = (10 + NW - 1) / NW;
    const int tp0 = (wave + 2) % NW;
    v4f graw[R], praw[R];

    // L (strict lower, beta) or Aqk (lower incl. diagonal) tile t of one value
    // head from its raw product; gt: that head's gc, beta
    auto scale_tile = [&](auto isPc, int t, const v4f &raw, const float *gt) {
        constexpr bool isP = decltype(isPc)::value;
        int ti, tj;
        lower_tile(t, ti, tj);
        // (the lane indices laundered: the index arithmetic is redone here
        // rather than kept alive from the first value head's call)
        int g4 = lane / 16, l16 = lane % 16;
        asm volatile("" : "+v"(g4), "+v"(l16));
        const float4 gr = *reinterpret_cast<const float4 *>(gt + 16 * ti + 4 * g4);
        const float gcol = gt[16 * tj + l16];
        float4 br = make_float4(1.f, 1.f, 1.f, 1.f);
        if (!isP) br = *reinterpret_cast<const float4 *>(gt + C + 16 * ti + 4 * g4);
        const float grr[4] = {gr.x, gr.y, gr.z, gr.w}, brr[4] = {br.x, br.y, br.z, br.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 16 * ti + 4 * g4 + r, col = 16 * tj + l16;
            // gc falls along the chunk, so the exponent is <= 0 where used
            const float e = expf(fminf(grr[r] - gcol, 0.f));
            if (isP) As[row * PC + col] = col <= row ? raw[r] * e : 0.f;
            else Ls[row * PC + col] = col < row ? brr[r] * raw[r] * e : 0.f;
        }
    };
    auto scale_all = [&](auto isPc, const float *gt) {
        constexpr bool isP = decltype(isPc)::value;
#pragma unroll
        for (int k = 0; k < R; k++) {
            const int t = (isP ? tp0 : wave) + NW * k;
            if (t < 10) scale_tile(isPc, t, isP ? praw[k] : graw[k], gt);
        }
    };

    // G = K K^T or P = Q K^T tile t: lane group g4 sums the contiguous k
    // range [g4 D/4, (g4+1) D/4), so operands load as float4
    auto product = [&](auto isPc, int t) {
        constexpr bool isP = decltype(isPc)::value;
        int ti, tj;
        lower_tile(t, ti, tj);
        const float *aa = (isP ? Qs : Ks) + (16 * ti + l16) * PD + g4 * (D / 4);
        const float *kb = Ks + (16 * tj + l16) * PD + g4 * (D / 4);
        v4f acc = v4zero(), acc2 = v4zero();
        // operands in groups of up to four float4 pairs (bounded registers)
        constexpr int NS4 = D / 16, GS = NS4 < 2 ? NS4 : 2;
#pragma unroll
        for (int s0 = 0; s0 < NS4; s0 += GS) {
            float4 A[GS], B[GS];
#pragma unroll
            for (int q = 0; q < GS; q++) {
                A[q] = *reinterpret_cast<const float4 *>(aa + 4 * (s0 + q));
                B[q] = *reinterpret_cast<const float4 *>(kb + 4 * (s0 + q));
            }
#pragma unroll
            for (int q = 0; q < GS; q++) {
                acc = mfma4(A[q].x, B[q].x, acc);
                acc2 = mfma4(A[q].y, B[q].y, acc2);
                acc = mfma4(A[q].z, B[q].z, acc);
                acc2 = mfma4(A[q].w, B[q].w, acc2);
            }
        }
        return acc + acc2;
    };

    // the diagonal blocks D_b = (I + L_bb)^-1 on the matrix cores (waves 0-3)
    auto inverses = [&]() {
        if (wave < 4) {
            const int b0 = 16 * wave;
            v4f nd;
#pragma unroll
            for (int r = 0; r < 4; r++) nd[r] = Ls[(b0 + 4 * g4 + r) * PC + b0 + l16];
            const v4f nt = *reinterpret_cast<const v4f *>(Ls + (b0 + l16) * PC + b0 + 4 * g4);
            const v4f xt = inv_unit_lower16(nd, nt, lane);
            *reinterpret_cast<v4f *>(Xs + (b0 + l16) * PC + b0 + 4 * g4) = xt;   // row l16 of D_b
        }
    };
    // the Aqk panel of (value head, chunk) hc from As, on the panel-writing
    // waves (4.. if there are more than four, else all)
    constexpr int PW = NW > 4 ? NW - 4 : NW;
    const int pw_t = NW > 4 ? tid - 4 * OMH_WAVE : tid;
    auto aqk_panel = [&](size_t hc) {
        if (pw_t >= 0)
            for (int e = pw_t; e < 16 * OMH_WAVE; e += PW * OMH_WAVE) {
                const int l = e % OMH_WAVE, kt = (e / OMH_WAVE) % 4, mt = e / (4 * OMH_WAVE);
                const int row = 16 * mt + l % 16, col = 16 * kt + 4 * (l / 16);
                *reinterpret_cast<float4 *>(a.pa + pan4(hc * 4 + mt, kt, l)) =
                    *reinterpret_cast<const float4 *>(As + row * PC + col);
            }
    };

    // W and U of (value head, chunk) hc by blocked forward substitution on
    // (I + L) [W | U] = [K beta e^gc | V beta], one 16-column tile per chain:
    //   R_i = D_i (RHS_i - sum_{k<i} L_ik R_k),
    // the tiles in registers in MFMA D layout (a D-layout tile feeds the B
    // operand directly: at k-step s lane group g supplies row 4g+s), each
    // R_k subtracted from every later row tile as soon as it is known.  With
    // D/16 waves each takes the W and the U chain of one column tile; with
    // fewer columns, one chain each.  U goes straight to its panel (the
    // scan's D layout); W is transposed through the wave's own columns of Qs
    // (no other wave reads them now) into the W panel's fragment order.
    auto substitution = [&](size_t hc, const float *gt) {
        constexpr bool TWO = NCT == NW;
        constexpr int NCH = TWO ? 2 : 1;
        const int q = wave;
        if (TWO || q < 2 * NCT) {
            const int tn = TWO ? q : q % NCT;
            const bool onlyU = !TWO && q >= NCT;
            v4f R[NCH][4];
            // right-hand sides (chain 0: W or U; chain 1: U)
#pragma unroll
            for (int ch = 0; ch < NCH; ch++) {
                const bool isU = ch == 1 || onlyU;
                const float *src = (isU ? Vs : Ks) + 16 * tn + l16;
                const float *scl = gt + (isU ? C : 2 * C) + 4 * g4;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 sv = *reinterpret_cast<const float4 *>(scl + 16 * i);
                    R[ch][i][0] = src[(16 * i + 4 * g4 + 0) * PD] * sv.x;
                    R[ch][i][1] = src[(16 * i + 4 * g4 + 1) * PD] * sv.y;
                    R[ch][i][2] = src[(16 * i + 4 * g4 + 2) * PD] * sv.z;
                    R[ch][i][3] = src[(16 * i + 4 * g4 + 3) * PD] * sv.w;
                }
            }
            v4f Xd[4], Ln[6];        // D_i and -L_ik (k < i) as A operands
#pragma unroll
            for (int i = 0; i < 4; i++) Xd[i] = *reinterpret_cast<const v4f *>(Xs + (16 * i + l16) * PC + 16 * i + 4 * g4);
#pragma unroll
            for (int i = 1, n = 0; i < 4; i++)
#pragma unroll
                for (int k = 0; k < i; k++, n++)
                    Ln[n] = -*reinterpret_cast<const v4f *>(Ls + (16 * i + l16) * PC + 16 * k + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int ch = 0; ch < NCH; ch++) R[ch][i] = mm16(Xd[i], R[ch][i], v4zero());
#pragma unroll
                for (int i2 = i + 1; i2 < 4; i2++)
#pragma unroll
                    for (int ch = 0; ch < NCH; ch++) R[ch][i2] = mm16(Ln[i2 * (i2 - 1) / 2 + i], R[ch][i], R[ch][i2]);
            }
            // U panel of column block tn, token tile i (the D layout of R)
            if (TWO || onlyU)
#pragma unroll
                for (int i = 0; i < 4; i++) *reinterpret_cast<v4f *>(a.pu + pan4(hc * NCT + tn, i, lane)) = R[NCH - 1][i];
            if (TWO || !onlyU) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) Qs[(16 * i + 4 * g4 + r) * PD + 16 * tn + l16] = R[0][i][r];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // W panel, k-group tn of token tile tt
#pragma unroll
                for (int tt = 0; tt < 4; tt++)
                    *reinterpret_cast<float4 *>(a.pw + panj<D>(hc, tt, tn, lane)) =
                        *reinterpret_cast<const float4 *>(Qs + (16 * tt + l16) * PD + 16 * tn + 4 * g4);
            }
        }
    };

    for (; m < nitems; m += gridDim.x) {
        int hk, h0, c, grp;
        wy_item(m, nitems, kh, rep, vpg, hk, h0, c, grp);
        const size_t hc0 = (size_t)h0 * nc + c, hc1 = hc0 + nc;   // value heads h0, h0 + 1
        const int m2 = m + (int)gridDim.x;
        const bool more = m2 < nitems;
        int hk2 = 0, h02 = 0, c2 = 0, grp2 = 0;
        if (more) wy_item(m2, nitems, kh, rep, vpg, hk2, h02, c2, grp2);

        // 1. this item's q, k, v0 and gates (computed during the item
        // before) into LDS; the next item's inputs start loading, spread
        // over phases 1-3 (and 6 for the second value head's v) so the
        // misses of one burst are in flight while the next phase computes
        in.template store<0, 3>(tid, Qs, Ks, Vs);
        if (gate) in.store_gates(a, gj == 0 ? hc0 : hc1, lane, gts + 3 * C * gj);
        if (more) in.template load<0, 1>(a, vpg, h02, hk2, c2, tid, gj, gate, lane, ph);
        omh_lds_barrier();

        // 2. L2 norm per token over the head's D channels (eps 1e-6), q also
        // scaled by D^-1/2 (qwen.c:153-157, 326-329)
        {
            // TPR consecutive lanes per row, each over D/TPR columns
            constexpr int TPR = WS::NT / (2 * C) >= 4 ? 4 : 2;
            constexpr int EPT = D / TPR;
            static_assert(EPT % 4 == 0 && WS::NT / TPR >= 2 * C / 2, "norm layout");
            for (int r = tid / TPR; r < 2 * C; r += WS::NT / TPR) {
                float *row = (r < C ? Qs + r * PD : Ks + (r - C) * PD) + (tid % TPR) * EPT;
                float4 v[EPT / 4];
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < EPT / 4; i++) {
                    v[i] = *reinterpret_cast<const float4 *>(row + 4 * i);
                    ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
                }
                ss = omh_group_sum<TPR>(ss);
                const float rr = 1.f / sqrtf(ss + 1e-6f);
                const float sc = 1.f / sqrtf((float)D);
#pragma unroll
                for (int i = 0; i < EPT / 4; i++) {
                    float4 y = f4_scale(v[i], rr);
                    if (r < C) y = f4_scale(y, sc);
                    *reinterpret_cast<float4 *>(row + 4 * i) = y;
                }
            }
        }
        if (more) in.template load<1, 2>(a, vpg, h02, hk2, c2, tid, gj, false, lane, ph);
        omh_lds_barrier();

        // 3. the products, kept raw for every value head; L and Aqk of value
        // head 0.  Each product shares a basic block with one conv unit of
        // the next item, so the conv's VALU work can issue between the MFMAs.
        if (more) in.template load<2, 3>(a, vpg, h02, hk2, c2, tid, gj, false, lane, ph);
        static_for<R>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int tg = wave + NW * k, tq = tp0 + NW * k;
            if (tg < 10) {
                graw[k] = product(std::false_type{}, tg);
                if (2 * k < 3) in.template compute_unit<(2 * k < 3 ? 2 * k : 0)>(a, c2, tid);
                scale_tile(std::false_type{}, tg, graw[k], gts);
            } else if (2 * k < 3) {
                in.template compute_unit<(2 * k < 3 ? 2 * k : 0)>(a, c2, tid);
            }
            if (tq < 10) {
                praw[k] = product(std::true_type{}, tq);
                if (2 * k + 1 < 3) in.template compute_unit<(2 * k + 1 < 3 ? 2 * k + 1 : 0)>(a, c2, tid);
                scale_tile(std::true_type{}, tq, praw[k], gts);
            } else if (2 * k + 1 < 3) {
                in.template compute_unit<(2 * k + 1 < 3 ? 2 * k + 1 : 0)>(a, c2, tid);
            }
        });
        static_assert(2 * R >= 3, "every conv unit has a slot");
        omh_lds_barrier();

        // 4. value head 0: the diagonal inverses on waves 0-3 while the
        // other waves write the q^ / k^T panels (once per key head: by the
        // first group's item) and the Aqk panel
        inverses();
        if (pw_t >= 0 && grp == 0) {
            // q^ / k^T panels (NST kd tiles x 4 token tiles x 64 lanes)
            const size_t hq = (size_t)hk * nc + c;
            for (int e = pw_t; e < NST * 4 * OMH_WAVE; e += PW * OMH_WAVE) {
                const int l = e % OMH_WAVE, tt = (e / OMH_WAVE) % 4, w = e / (4 * OMH_WAVE);
                const int ll16 = l % 16, lg = l / 16;
                const int rq = tt * 16 + ll16, cq = 16 * w + 4 * lg;
                const float4 vq = *reinterpret_cast<const float4 *>(Qs + rq * PD + cq);
                const int rk = tt * 16 + 4 * lg, ck = 16 * w + ll16;
                const float4 vk =
                    make_float4(Ks[rk * PD + ck], Ks[(rk + 1) * PD + ck], Ks[(rk + 2) * PD + ck], Ks[(rk + 3) * PD + ck]);
                *reinterpret_cast<float4 *>(a.pq + panj<D>(hq, tt, w, l)) = vq;
                *reinterpret_cast<float4 *>(a.pk + pan4(hq * NST + w, tt, l)) = vk;
            }
        }
        aqk_panel(hc0);
        omh_lds_barrier();

        // 5. value head 0: W and U; the gates of the next item
        substitution(hc0, gts);
        if (gate) in.gates(a, h02 + gj, c2, lane);
        omh_lds_barrier();

        if (vpg == 2) {
            // 6. value head 1: L, Aqk (nothing reads Ls, As now) and v into LDS
            scale_all(std::false_type{}, gts + 3 * C);
            scale_all(std::true_type{}, gts + 3 * C);
            in.template store<3, 4>(tid, Qs, Ks, Vs);
            omh_lds_barrier();
            // 7. value head 1: inverses and the Aqk panel; the next item's v
            // of its second value head starts loading
            if (more) in.template load<3, 4>(a, vpg, h02, hk2, c2, tid, gj, false, lane, ph);
            inverses();
            aqk_panel(hc1);
            omh_lds_barrier();
            // 8. value head 1: W and U; the next item's second v conv
            substitution(hc1, gts + 3 * C);
            in.template compute_unit<3>(a, c2, tid);
            omh_lds_barrier();
        }
    }
}

// ---------------------------------------------------------------- P3 scan
// One chunk's operands for one scan wave, in MFMA fragment order: for a
// v_new wave (V = true) the W and U tiles of its token tile and e^{gl-gc} of
// its rows, for an output wave the q^ and Aqk tiles and e^gc of its rows;
// for both the k^T row tile of the S tile the wave holds, and e^{gl}.
// Loaded in parts (load_m, load_x, load_k) so each part can be spread over a
// different product.
template <int D, bool V>
struct ScanIn {
    static constexpr int NST = ScanShape<D>::NST;
    static constexpr int NX = V ? 4 : 16;
    float Mf[4 * NST];   // W or q^, token tile w % 4
    float Xf[NX];        // U tile (D layout) or Aqk row tile
    float Kf[16];        // k^T of row tile w
    float sc[4];         // e^{gl-gc} (v_new waves) or e^gc (output waves) of rows 4g..4g+3 of token tile w % 4
    float eg;            // e^{gl}

    // hc: (value head, chunk); hq: (key head, chunk)
    __device__ __forceinline__ void load_m(const PrefillArgs &a, size_t hc, size_t hq, int w, int lane) {
        const float *mp = V ? a.pw + panj<D>(hc, w & 3, 0, lane) : a.pq + panj<D>(hq, w & 3, 0, lane);
#pragma unroll
        for (int kt = 0; kt < NST; kt++) {
            const float4 x = *reinterpret_cast<const float4 *>(mp + kt * OMH_WAVE * 4);
            Mf[4 * kt] = x.x; Mf[4 * kt + 1] = x.y; Mf[4 * kt + 2] = x.z; Mf[4 * kt + 3] = x.w;
        }
    }
    __device__ __forceinline__ void load_x(const PrefillArgs &a, size_t hc, int cb, int w, int lane) {
        const float *xp = V ? a.pu + pan4(hc * (D / 16) + cb, w & 3, lane) : a.pa + pan4(hc * 4 + (w & 3), 0, lane);
#pragma unroll
        for (int kt = 0; kt < NX / 4; kt++) {
            const float4 x = *reinterpret_cast<const float4 *>(xp + kt * OMH_WAVE * 4);
            Xf[4 * kt] = x.x; Xf[4 * kt + 1] = x.y; Xf[4 * kt + 2] = x.z; Xf[4 * kt + 3] = x.w;
        }
        const float4 x = *reinterpret_cast<const float4 *>((V ? a.pe : a.pg) + hc * C + 16 * (w & 3) + 4 * (lane / 16));
        sc[0] = x.x; sc[1] = x.y; sc[2] = x.z; sc[3] = x.w;
    }
    // eg comes through a buffer load (a vector load at a uniform offset): a
    // scalar load would share lgkmcnt with the LDS reads and hold them up.
    __device__ __forceinline__ void load_k(const PrefillArgs &a, __amdgpu_buffer_rsrc_t grs, size_t hc, size_t hq, int w,
                                           int lane) {
        const float *kp = a.pk + pan4(hq * NST + (w < NST ? w : NST - 1), 0, lane);
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const float4 x = *reinterpret_cast<const float4 *>(kp + tt * OMH_WAVE * 4);
            Kf[4 * tt] = x.x; Kf[4 * tt + 1] = x.y; Kf[4 * tt + 2] = x.z; Kf[4 * tt + 3] = x.w;
        }
        eg = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(grs, 0, (int)(hc * 4), 0));
    }
};

// LDS of one scan workgroup (each tile is only ever read as the B operand
// of a product)
template <int D>
struct ScanLds {
    v4f S[ScanShape<D>::NST][OMH_WAVE];      // S row tiles at the start of the chunk
    v4f V[4][OMH_WAVE];                      // v_new token tiles
    v4f Vs[4][OMH_WAVE];                     // the same rows scaled by e^{gl-gc}
    __device__ __forceinline__ static v4f put(v4f x) { return x; }
};

// c + (16 x 16 A fragment held as four k-step values a[0..3]) x (B tile of
// one k-step group): four fp32 products
__device__ __forceinline__ v4f mm4(const float *a, const v4f &b, v4f c) {
#pragma unroll
    for (int s = 0; s < 4; s++) c = mfma4(a[s], b[s], c);
    return c;
}

// S <- e^{gl} S + (K e^{gl-gc})^T v_new for the wave's row tile (two chains)
template <int D, bool V>
__device__ __forceinline__ void scan_update_s(const ScanIn<D, V> &f, const v4f (&VN)[4], v4f &S) {
    v4f S2 = v4zero();
    S *= f.eg;
#pragma unroll
    for (int tt = 0; tt < 4; tt += 2) {
        S = mm4(f.Kf + tt * 4, VN[tt], S);
        S2 = mm4(f.Kf + (tt + 1) * 4, VN[tt + 1], S2);
    }
    S += S2;
}

// (token tile) x S over all of kd: the B operand of k-step (kt, s) is
// register s of S row tile kt (D layout), read from LDS; two chains
template <int D, bool V>
__device__ __forceinline__ void scan_times_s(const ScanIn<D, V> &f, const v4f (&Ss)[ScanShape<D>::NST][OMH_WAVE], int lane,
                                             v4f &P0, v4f &P1) {
#pragma unroll
    for (int kt = 0; kt < ScanShape<D>::NST; kt++) {
        const v4f sf = Ss[kt][lane];
        if (kt & 1) P1 = mm4(f.Mf + kt * 4, sf, P1);
        else P0 = mm4(f.Mf + kt * 4, sf, P0);
    }
}

// Instruction order for a product over NST row tiles read from LDS, with NL
// of the next chunk's loads spread over its MFMAs (the L1 return path then
// works while the matrix cores do, instead of every wave queueing its loads
// at once).  MPK: MFMAs per row tile.
template <int NST, int NL, int MPK = 4>
__device__ __forceinline__ void scan_interleave_s() {
    constexpr int PER = (NL + NST - 1) / NST;
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);        // first S tiles
#pragma unroll
    for (int kt = 0; kt < NST; kt++) {
        __builtin_amdgcn_sched_group_barrier(0x008, MPK, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, PER, 0);  // loads
        if (kt + 2 < NST) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}
// NM MFMAs (operands in registers) with NL loads spread over them
template <int NM, int NL>
__device__ __forceinline__ void scan_interleave_r() {
    constexpr int PER = (NM + NL - 1) / NL;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
}

// Per (value head, 16-column block of S): the chunk recurrence, S held in
// registers (MFMA D layout, one 16-row tile per wave w < D/16) for the whole
// sequence.  Per chunk, two barriers:
//   B1: every S row tile of the chunk is in LDS.  Waves 0-3 each form
//       v_new = U - W S for one token tile (contracting over all of kd) into
//       LDS, once as is and once with its rows scaled by e^{gl-gc}; waves 4-7
//       each form e^gc (q^ S) for one token tile.
//   B2: v_new is in LDS.  Every wave updates its S tile,
//       S <- e^{gl} S + k^T (e^{gl-gc} v_new), and writes it to LDS for the
//       next chunk; waves 4-7 add Aqk v_new over all key tiles (the panel's
//       tiles above the diagonal are zero) to finish their output tile,
//       which they store after the next B1.
// Each matrix core then has 64 MFMAs before B2 (W S and Q S) and 48 after.
// The two roles run separate loops with the same barriers; each loads the
// operands of the chunk after next into a third register set (two chunks of
// lead time for HBM latency), spread over its own products.
template <int D>
__global__ __launch_bounds__((ScanShape<D>::NWV * OMH_WAVE), 1)
void prefill_scan_kernel(const PrefillArgs a) {
    constexpr int NST = ScanShape<D>::NST;
    constexpr int NCB = D / 16;
    const int vh = a.vh;
    // XCD-aware: the column blocks of all value heads of a key head share one
    // XCD (and its L2), so the key head's q^ / k^ panels are fetched once
    const int rep = vh / a.kh;
    int h, cb;
    {
        const int n = blockIdx.x;
        if (a.kh % 8 == 0) {
            const int x = n % 8, m = n / 8;
            h = (x + 8 * (m / (rep * NCB))) * rep + (m / NCB) % rep;
            cb = m % NCB;
        } else {
            h = n / NCB;
            cb = n % NCB;
        }
    }
    const int hk = h / rep;
    const size_t hq0 = (size_t)hk * a.nc;
    const int lane = threadIdx.x % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / OMH_WAVE);
    const int l16 = lane % 16, g4 = lane / 16;
    const int j = w & 3;                 // token tile of the wave's job
    const bool owns = w < NST;           // holds S row tile w
    const int nc = a.nc;
    const size_t hc0 = (size_t)h * nc;
    const __amdgpu_buffer_rsrc_t grs =
        __builtin_amdgcn_make_buffer_rsrc(a.glast, 0, (int)((size_t)vh * nc * sizeof(float)), 0x00020000);

    using Lds = ScanLds<D>;
    constexpr int MPK = 4;                               // MFMAs per 16x16x16 step
    __shared__ Lds sm;

    // S rows 16w + 4g + r, column 16cb + l%16
    float *Sbase = a.L.S + ((size_t)a.seq * vh + h) * (D * D);
    v4f S = v4zero();
    if (owns) {
#pragma unroll
        for (int r = 0; r < 4; r++) S[r] = Sbase[(size_t)(16 * w + 4 * g4 + r) * D + 16 * cb + l16];
        sm.S[w][lane] = Lds::put(S);
    }

    if (w < 4) {
        // v_new waves
        typedef ScanIn<D, true> In;
        auto step = [&](const In &f, In &fn, int c) {
            const int cn = min(c + 2, nc - 1);
            omh_lds_barrier();                   // B1: S tiles of chunk c
            fn.load_m(a, hc0 + cn, hq0 + cn, w, lane);
            v4f P0 = v4zero(), P1 = v4zero();
            scan_times_s<D, true>(f, sm.S, lane, P0, P1);
            scan_interleave_s<NST, NST, MPK>();
            v4f vn, vs;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                vn[r] = f.Xf[r] - (P0[r] + P1[r]);
                vs[r] = vn[r] * f.sc[r];
            }
            sm.V[j][lane] = Lds::put(vn);
            sm.Vs[j][lane] = Lds::put(vs);
            omh_lds_barrier();                   // B2: v_new of chunk c
            fn.load_x(a, hc0 + cn, cb, w, lane);
            fn.load_k(a, grs, hc0 + cn, hq0 + cn, w, lane);
            if (owns) {
                v4f VN[4];
#pragma unroll
                for (int tt = 0; tt < 4; tt++) VN[tt] = sm.Vs[tt][lane];
                scan_update_s<D, true>(f, VN, S);
                scan_interleave_r<4 * MPK, 7>();
                sm.S[w][lane] = Lds::put(S);
            }
        };
        In f0, f1, f2;
        const int c1 = min(1, nc - 1);
        f0.load_m(a, hc0, hq0, w, lane);
        f0.load_x(a, hc0, cb, w, lane);
        f0.load_k(a, grs, hc0, hq0, w, lane);
        f1.load_m(a, hc0 + c1, hq0 + c1, w, lane);
        f1.load_x(a, hc0 + c1, cb, w, lane);
        f1.load_k(a, grs, hc0 + c1, hq0 + c1, w, lane);
        for (int c = 0; c < nc; c += 3) {
            step(f0, f2, c);
            if (c + 1 < nc) step(f1, f0, c + 1);
            if (c + 2 < nc) step(f2, f1, c + 2);
        }
    } else {
        // output waves
        typedef ScanIn<D, false> In;
        float *obase = a.core + (size_t)h * D + 16 * cb + l16;
        const size_t vdim = (size_t)vh * D;
        v4f o = v4zero();
        auto store = [&](int c) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = c * C + 16 * j + 4 * g4 + r;
                if (t < a.T) obase[(size_t)t * vdim] = o[r];
            }
        };
        auto step = [&](const In &f, In &fn, int c) {
            const int cn = min(c + 2, nc - 1);
            omh_lds_barrier();                   // B1: S tiles of chunk c
            if (c > 0) store(c - 1);
            fn.load_m(a, hc0 + cn, hq0 + cn, w, lane);
            fn.load_x(a, hc0 + cn, cb, w, lane);
            v4f O0 = v4zero(), O1 = v4zero();
            scan_times_s<D, false>(f, sm.S, lane, O0, O1);
            scan_interleave_s<NST, NST + 5, MPK>();
#pragma unroll
            for (int r = 0; r < 4; r++) O0[r] = (O0[r] + O1[r]) * f.sc[r];
            O1 = v4zero();
            omh_lds_barrier();                   // B2: v_new of chunk c
            fn.load_k(a, grs, hc0 + cn, hq0 + cn, w, lane);
            if (owns) {
                v4f VS[4];
#pragma unroll
                for (int tt = 0; tt < 4; tt++) VS[tt] = sm.Vs[tt][lane];
                scan_update_s<D, false>(f, VS, S);
                sm.S[w][lane] = Lds::put(S);
            }
            v4f VN[4];
#pragma unroll
            for (int tt = 0; tt < 4; tt++) VN[tt] = sm.V[tt][lane];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                if (kt & 1) O1 = mm4(f.Xf + kt * 4, VN[kt], O1);
                else O0 = mm4(f.Xf + kt * 4, VN[kt], O0);
            }
            scan_interleave_r<8 * MPK, 5>();
            o = O0 + O1;
        };
        In f0, f1, f2;
        const int c1 = min(1, nc - 1);
        f0.load_m(a, hc0, hq0, w, lane);
        f0.load_x(a, hc0, cb, w, lane);
        f0.load_k(a, grs, hc0, hq0, w, lane);
        f1.load_m(a, hc0 + c1, hq0 + c1, w, lane);
        f1.load_x(a, hc0 + c1, cb, w, lane);
        f1.load_k(a, grs, hc0 + c1, hq0 + c1, w, lane);
        for (int c = 0; c < nc; c += 3) {
            step(f0, f2, c);
            if (c + 1 < nc) step(f1, f0, c + 1);
            if (c + 2 < nc) step(f2, f1, c + 2);
        }
        store(nc - 1);
    }
    if (owns)
#pragma unroll
        for (int r = 0; r < 4; r++) Sbase[(size_t)(16 * w + 4 * g4 + r) * D + 16 * cb + l16] = S[r];
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workgroups of the persistent WY kernel: the device's CU count.
int wy_grid() {
    static int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
            cus = 256;
        return cus - cus % 8;
    }();
    return n;
}

template <int D>
hipError_t launch_prefill_d(const PrefillArgs &a, hipStream_t st) {
    const int conv_dim = 2 * a.kh * D + a.vh * D;
    // persistent: one workgroup per CU (the LDS footprint allows one), a
    // multiple of 8 so the XCD-aware item order holds
    const int rep = a.vh / a.kh;
    const int nitems = a.kh * (rep % 2 == 0 ? rep / 2 : rep) * a.nc;   // as in the kernel
    const int grid = nitems < wy_grid() ? nitems : wy_grid();
    // the WY kernel reads the ring for chunk 0 before the commit (in the
    // norm launch) rewrites it
    if (a.K == 4) hipLaunchKernelGGL((prefill_wy_kernel<D, 4>), dim3(grid), dim3(WyShape<D>::NT), WyShape<D>::LDS, st, a);
    else if (a.K == 3) hipLaunchKernelGGL((prefill_wy_kernel<D, 3>), dim3(grid), dim3(WyShape<D>::NT), WyShape<D>::LDS, st, a);
    else hipLaunchKernelGGL((prefill_wy_kernel<D, 2>), dim3(grid), dim3(WyShape<D>::NT), WyShape<D>::LDS, st, a);
    hipLaunchKernelGGL((prefill_scan_kernel<D>), dim3(a.vh * (D / 16)), dim3(ScanShape<D>::NWV * OMH_WAVE), 0, st, a);
    constexpr int RPB = 256 / (D / 4);
    const size_t rows = (size_t)a.T * a.vh;
    const int nnorm = (int)((rows + RPB - 1) / RPB), ncommit = (conv_dim + 255) / 256;
    hipLaunchKernelGGL((prefill_gated_norm_kernel<D>), dim3((unsigned)(nnorm + ncommit)), dim3(256), 0, st, a, nnorm,
                       conv_dim);
    return hipGetLastError();
}

template <int D>
bool set_lds_limit() {
    bool ok = true;
    for (const void *f : {(const void *)prefill_wy_kernel<D, 2>, (const void *)prefill_wy_kernel<D, 3>,
                          (const void *)prefill_wy_kernel<D, 4>})
        ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)WyShape<D>::LDS) == hipSuccess;
    return ok;
}

}  // namespace

size_t prefill_scratch_bytes(int D, int kh, int vh, int T) {
    const size_t Tp = (size_t)((T + C - 1) / C) * C, nc = Tp / C;
    size_t n = 0;
    n += align256((size_t)vh * nc * 4);                    // glast
    n += 2 * align256((size_t)vh * Tp * 4);                // pg, pe
    n += align256((size_t)vh * Tp * D * 4);                // pw
    n += 2 * align256((size_t)kh * Tp * D * 4);            // pq, pk
    n += align256((size_t)vh * nc * C * C * 4);            // pa
    n += align256((size_t)vh * Tp * D * 4);                // pu
    return n;
}

void prefill_bind_scratch(PrefillArgs &a, int D, void *base) {
    const size_t Tp = (size_t)a.Tp, nc = (size_t)a.nc;
    char *p = static_cast<char *>(base);
    auto take = [&](size_t bytes) { float *r = reinterpret_cast<float *>(p); p += align256(bytes); return r; };
    a.glast = take((size_t)a.vh * nc * 4);
    a.pg = take((size_t)a.vh * Tp * 4);
    a.pe = take((size_t)a.vh * Tp * 4);
    a.pw = take((size_t)a.vh * Tp * D * 4);
    a.pq = take((size_t)a.kh * Tp * D * 4);
    a.pk = take((size_t)a.kh * Tp * D * 4);
    a.pa = take((size_t)a.vh * nc * C * C * 4);
    a.pu = take((size_t)a.vh * Tp * D * 4);
}

bool prefill_supported(int kd, int vd, int rep, int K) {
    if (rep < 1 || K < 2 || K > kConvRing || kd != vd) return false;
    return kd == 16 || kd == 32 || kd == 64 || kd == 128;
}

hipError_t launch_prefill_core(const PrefillArgs &a, int D, hipStream_t st) {
    static bool lds_ok = set_lds_limit<16>() && set_lds_limit<32>() && set_lds_limit<64>() && set_lds_limit<128>();
    if (!lds_ok) return hipErrorInvalidValue;
    switch (D) {
        case 16: return launch_prefill_d<16>(a, st);
        case 32: return launch_prefill_d<32>(a, st);
        case 64: return launch_prefill_d<64>(a, st);
        case 128: return launch_prefill_d<128>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace omh
