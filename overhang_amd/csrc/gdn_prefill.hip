// gdn_prefill.hip — chunked (WY/UT) prefill of T tokens of one sequence.
//
// Same recurrence as the decode path (overhang engines/qwen.c:307-358, one
// token at a time there), evaluated chunk-wise as transformers'
// torch_chunk_gated_delta_rule does (modeling_qwen3_5_moe.py:250-328):
// for a chunk of C = 64 tokens with cumulative log-decay gc,
//     L  = strict_lower(beta_i k_i.k_j exp(gc_i - gc_j)),   X = (I + L)^-1
//     W  = X (K * beta * e^gc),   U = X (V * beta)
//     Aqk = lower_incl_diag(q_i.k_j exp(gc_i - gc_j))
//     v_new = U - W S;   o = (Q * e^gc) S + Aqk v_new
//     S <- e^{gc_last} S + (K * e^{gc_last - gc})^T v_new
// Only exp of differences of cumulative decays are formed, never exp(-gc).
//
// Five launches, all on the caller's stream:
//   P1 prep    conv + SiLU, q/k L2 norm (+ q scale), gates        HBM-bound
//   P5 commit  conv history ring -> last K-1 inputs, new phase     tiny
//   P2 chunk   per (value head, chunk): KK^T, QK^T, X, W, U on fp32 MFMA,
//              written as per-lane fragment panels for P3          MFMA-bound
//   P3 scan    per (value head, 16-column block): the chunk recurrence,
//              sequential over chunks, on fp32 MFMA                MFMA-bound
//   P4 norm    gated RMSNorm of the head outputs                   HBM-bound
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

namespace omh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int C = kChunk;

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f v4zero() { v4f z = {0.f, 0.f, 0.f, 0.f}; return z; }

// Scan work split for head dim D: NWV waves per workgroup, each owning KT
// kd tiles of S and TT of the chunk's 4 token tiles.
template <int D>
struct ScanShape {
    static constexpr int NWV = D / 16 < 4 ? D / 16 : 4;
    static constexpr int KT = D / 16 / NWV;
    static constexpr int TT = 4 / NWV;
    static constexpr int NFW = 16 * KT;        // W / Q fragments per lane per chunk
    static constexpr int NFK = 16 * KT;        // K^T fragments
    static constexpr int NFA = 16 * TT;        // Aqk fragments
    static constexpr int NFU = 4 * TT;         // U values per column block
    static_assert(NWV * KT * 16 == D && NWV * TT == 4, "scan split");
};

// ---------------------------------------------------------------- P1 prep
// grid (2*kh + vh, Tp/C); thread = channel of one q, k or v head.
template <int D>
__global__ __launch_bounds__((D < 64 ? 64 : D))
void prefill_prep_kernel(const PrefillArgs a) {
    constexpr int NT = D < 64 ? 64 : D;
    constexpr int NW = NT / OMH_WAVE;
    const int grp = blockIdx.x, t0 = blockIdx.y * C;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE, wave = tid / OMH_WAVE;
    const int kh = a.kh, vh = a.vh, K = a.K;
    const int key_dim = kh * D, conv_dim = 2 * key_dim + vh * D;
    int kind, head, gch0;
    if (grp < kh) { kind = 0; head = grp; gch0 = grp * D; }
    else if (grp < 2 * kh) { kind = 1; head = grp - kh; gch0 = key_dim + head * D; }
    else { kind = 2; head = grp - 2 * kh; gch0 = 2 * key_dim + head * D; }

    __shared__ float s_y[C][D + 1];
    if (tid < D) {
        const int gch = gch0 + tid;
        float w[kConvRing], h[kConvRing - 1];
        const float4 wv = *reinterpret_cast<const float4 *>(a.L.conv_w + (size_t)gch * kConvRing);
        for (int j = 0; j < K; j++) w[j] = f4_get(wv, j);
        if (t0 == 0) {
            const int ph = a.L.phase[a.L.epoch * a.L.max_seqs + a.seq];
            const float4 rv = *reinterpret_cast<const float4 *>(a.L.conv_st + ring_at(a.seq, gch, conv_dim));
            for (int j = 0; j < K - 1; j++) h[j] = f4_get(rv, ring_slot(ph, K, j));
        } else {
            for (int j = 0; j < K - 1; j++) h[j] = a.qkv[(size_t)(t0 - (K - 1) + j) * a.ld_qkv + gch];
        }
        float *vout = a.v + ((size_t)head * a.Tp + t0) * D + tid;
        for (int t = 0; t < C; t++) {
            const int tt = t0 + t;
            float y = 0.f;
            if (tt < a.T) {
                const float x = a.qkv[(size_t)tt * a.ld_qkv + gch];
                float acc = 0.f;
                for (int j = 0; j < K - 1; j++) acc += w[j] * h[j];   // qwen.c:315-316
                acc += w[K - 1] * x;
                for (int j = 0; j < K - 2; j++) h[j] = h[j + 1];
                h[K - 2] = x;
                y = omh_silu(acc);
            }
            if (kind == 2) vout[(size_t)t * D] = y;
            else s_y[t][tid] = y;
        }
    }
    if (kind == 2) {
        if (tid < C) {                            // gates (qwen.c:337-338)
            const int tt = t0 + tid;
            float g = 0.f, be = 0.f;
            if (tt < a.T) {
                g = -expf(a.L.A_log[head]) * omh_softplus(a.a[(size_t)tt * a.ld_ab + head] + a.L.dt_bias[head]);
                be = omh_sigmoid(a.b[(size_t)tt * a.ld_ab + head]);
            }
            a.g[(size_t)head * a.Tp + tt] = g;
            a.beta[(size_t)head * a.Tp + tt] = be;
        }
        return;
    }
    __syncthreads();
    // per-token L2 norm over the head's D channels (qwen.c:153-157, 327-329)
    float *out = (kind == 0 ? a.qn : a.kn) + ((size_t)head * a.Tp + t0) * D;
    const float scale = kind == 0 ? 1.f / sqrtf((float)D) : 1.f;
    for (int t = wave; t < C; t += NW) {
        float ss = 0.f;
        for (int i = lane; i < D; i += OMH_WAVE) ss += s_y[t][i] * s_y[t][i];
        ss = omh_xor_sum_below<OMH_WAVE>(ss);
        const float r = 1.f / sqrtf(ss + 1e-6f);
        for (int i = lane; i < D; i += OMH_WAVE) {
            const float q = s_y[t][i] * r;
            out[(size_t)t * D + i] = kind == 0 ? q * scale : q;
        }
    }
}

// ---------------------------------------------------------------- P5 commit
// New conv history = last K-1 entries of [old history, x_0 .. x_{T-1}],
// written in ring order for phase (p + T) mod ring size.  Every block reads
// the phase from phase[epoch]; the new one goes to phase[1 - epoch] (block 0
// also carries the other sequences' phases over) and the host flips the
// layer's epoch after the launch, as for decode launches.
__global__ __launch_bounds__(256)
void prefill_conv_commit_kernel(const PrefillArgs a, int conv_dim) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int K = a.K, T = a.T;
    const int ph = a.L.phase[a.L.epoch * a.L.max_seqs + a.seq];
    const int nph = (ph + T) & (kConvRing - 1);
    if (c < conv_dim) {
        float4 *ring = reinterpret_cast<float4 *>(a.L.conv_st + ring_at(a.seq, c, conv_dim));
        const float4 old = *ring;
        float4 e = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < K - 1; j++) {
            const int idx = T + j;               // index into [old history (K-1), x_0 ..]
            const float v = idx < K - 1 ? f4_get(old, ring_slot(ph, K, idx))
                                        : a.qkv[(size_t)(idx - (K - 1)) * a.ld_qkv + c];
            f4_set(e, ring_slot(nph, K, j), v);
        }
        *ring = e;
    }
    if (blockIdx.x == 0) {
        int *nxt = a.L.phase + (1 - a.L.epoch) * a.L.max_seqs;
        const int *cur = a.L.phase + a.L.epoch * a.L.max_seqs;
        for (int s = threadIdx.x; s < a.L.max_seqs; s += 256) nxt[s] = s == a.seq ? nph : cur[s];
    }
}

// ---------------------------------------------------------------- P4 norm
template <int D>
__global__ __launch_bounds__(256)
void prefill_gated_norm_kernel(const PrefillArgs a) {
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

// Panel addressing: frag f of lane l of wave w, in float4 groups so that a
// wave's consecutive lanes read consecutive 16 B.
__device__ __forceinline__ size_t panel_idx(size_t base4, int f, int l) {
    return ((base4 + (size_t)(f >> 2)) * OMH_WAVE + l) * 4 + (f & 3);
}

// ---------------------------------------------------------------- P2 chunk
template <int D>
__global__ __launch_bounds__(256)
void prefill_chunk_kernel(const PrefillArgs a) {
    using SS = ScanShape<D>;
    constexpr int NWV = SS::NWV, KT = SS::KT, TT = SS::TT;
    constexpr int PD = D + 4, PC = C + 4;        // padded LDS row lengths
    const int h = blockIdx.x, c = blockIdx.y;
    const int vh = a.vh, rep = vh / a.kh, hk = h / rep;
    const int t0 = c * C;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE, wave = tid / OMH_WAVE;
    const int l16 = lane % 16, g4 = lane / 16;

    extern __shared__ float smem[];
    float *Ks = smem;                            // [C][PD]
    float *Qs = Ks + C * PD;                     // [C][PD]
    float *Vs = Qs + C * PD;                     // [C][PD]
    float *Xs = Vs + C * PD;                     // [C][PC]  L, then X = (I+L)^-1
    float *As = Xs + C * PC;                     // [C][PC]  Aqk
    float *gcs = As + C * PC;                    // [C]
    float *bs = gcs + C;                         // [C]

    // 1. stage K, Q (key head hk), V (value head h), g, beta
    {
        const float *kp = a.kn + ((size_t)hk * a.Tp + t0) * D;
        const float *qp = a.qn + ((size_t)hk * a.Tp + t0) * D;
        const float *vp = a.v + ((size_t)h * a.Tp + t0) * D;
        for (int e = tid; e < C * D / 4; e += 256) {
            const int r = e / (D / 4), c4 = e % (D / 4);
            const float4 kk = *reinterpret_cast<const float4 *>(kp + (size_t)e * 4);
            const float4 qq = *reinterpret_cast<const float4 *>(qp + (size_t)e * 4);
            const float4 vv = *reinterpret_cast<const float4 *>(vp + (size_t)e * 4);
            float *kd = Ks + r * PD + c4 * 4, *qd = Qs + r * PD + c4 * 4, *vd = Vs + r * PD + c4 * 4;
            kd[0] = kk.x; kd[1] = kk.y; kd[2] = kk.z; kd[3] = kk.w;
            qd[0] = qq.x; qd[1] = qq.y; qd[2] = qq.z; qd[3] = qq.w;
            vd[0] = vv.x; vd[1] = vv.y; vd[2] = vv.z; vd[3] = vv.w;
        }
        if (wave == 0) {
            // inclusive prefix sum of g over the chunk (one lane per token)
            float x = a.g[(size_t)h * a.Tp + t0 + lane];
#pragma unroll
            for (int off = 1; off < OMH_WAVE; off <<= 1) {
                const float y = __shfl_up(x, off, OMH_WAVE);
                if (lane >= off) x += y;
            }
            gcs[lane] = x;
            bs[lane] = a.beta[(size_t)h * a.Tp + t0 + lane];
            if (lane == C - 1) a.glast[(size_t)h * a.nc + c] = expf(x);
        }
    }
    __syncthreads();

    // 2. G = K K^T and QK = Q K^T, lower tiles only; wave w owns row tile w
    {
        v4f G[4], Q[4];
#pragma unroll
        for (int n = 0; n < 4; n++) { G[n] = v4zero(); Q[n] = v4zero(); }
        const int m0 = wave * 16;
        for (int k0 = 0; k0 < D; k0 += 4) {
            const float ak = Ks[(m0 + l16) * PD + k0 + g4];
            const float aq = Qs[(m0 + l16) * PD + k0 + g4];
#pragma unroll
            for (int n = 0; n < 4; n++) {
                if (n <= wave) {
                    const float bk = Ks[(n * 16 + l16) * PD + k0 + g4];
                    G[n] = mfma4(ak, bk, G[n]);
                    Q[n] = mfma4(aq, bk, Q[n]);
                }
            }
        }
        // masks and decays; write full rows of the row tile
#pragma unroll
        for (int n = 0; n < 4; n++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int i = m0 + 4 * g4 + r, j = n * 16 + l16;
                float lv = 0.f, av = 0.f;
                if (j <= i) {
                    const float dec = expf(gcs[i] - gcs[j]);
                    av = Q[n][r] * dec;
                    if (j < i) lv = bs[i] * G[n][r] * dec;
                }
                Xs[i * PC + j] = lv;
                As[i * PC + j] = av;
            }
        }
    }
    __syncthreads();

    const size_t hc = (size_t)h * a.nc + c;
    if (wave == 0) {
        // 3a. X = (I + L)^-1 by forward substitution; lane j keeps column j
        // of X: X[i][j] = -sum_{m<i} L[i][m] X[m][j] for j < i, X[j][j] = 1.
        float xc[C];
#pragma unroll
        for (int i = 0; i < C; i++) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < i; m++) acc += Xs[i * PC + m] * xc[m];
            xc[i] = lane < i ? -acc : (lane == i ? 1.f : 0.f);
        }
#pragma unroll
        for (int i = 0; i < C; i++) Xs[i * PC + lane] = xc[i];
    } else {
        // 3b. panels that do not need X: Q*e^gc, (K*e^{gl-gc})^T, Aqk
        const float gl = gcs[C - 1];
        for (int e = tid - OMH_WAVE; e < NWV * OMH_WAVE * SS::NFW; e += 256 - OMH_WAVE) {
            const int f = e % SS::NFW, l = (e / SS::NFW) % OMH_WAVE, w = e / (SS::NFW * OMH_WAVE);
            const int ll16 = l % 16, lg = l / 16;
            // W/Q order: f = (tt*KT + kt)*4 + s -> row 16tt + l%16, col 16(w*KT+kt) + 4g + s
            {
                const int s = f & 3, kt = (f >> 2) % KT, tt = (f >> 2) / KT;
                const int row = tt * 16 + ll16, col = 16 * (w * KT + kt) + 4 * lg + s;
                a.pq[panel_idx((hc * NWV + w) * (SS::NFW / 4), f, l)] = Qs[row * PD + col] * expf(gcs[row]);
            }
            // K order: f = (kt*4 + tt)*4 + s -> row (token) 16tt + 4g + s, col 16(w*KT+kt) + l%16
            {
                const int s = f & 3, tt = (f >> 2) & 3, kt = f >> 4;
                const int row = tt * 16 + 4 * lg + s, col = 16 * (w * KT + kt) + ll16;
                a.pk[panel_idx((hc * NWV + w) * (SS::NFK / 4), f, l)] = Ks[row * PD + col] * expf(gl - gcs[row]);
            }
        }
        for (int e = tid - OMH_WAVE; e < NWV * OMH_WAVE * SS::NFA; e += 256 - OMH_WAVE) {
            // A order: f = u*16 + kt*4 + s -> row 16(w*TT+u) + l%16, col 16kt + 4g + s
            const int f = e % SS::NFA, l = (e / SS::NFA) % OMH_WAVE, w = e / (SS::NFA * OMH_WAVE);
            const int s = f & 3, kt = (f >> 2) & 3, u = f >> 4;
            const int row = 16 * (w * TT + u) + l % 16, col = 16 * kt + 4 * (l / 16) + s;
            a.pa[panel_idx((hc * NWV + w) * (SS::NFA / 4), f, l)] = As[row * PC + col];
        }
    }
    __syncthreads();

    // 4. W = X (K * beta * e^gc), U = X (V * beta); wave w owns token tile w
    constexpr int NT16 = D / 16;
    v4f Wt[NT16], Ut[NT16];
#pragma unroll
    for (int n = 0; n < NT16; n++) { Wt[n] = v4zero(); Ut[n] = v4zero(); }
    {
        const int m0 = wave * 16;
        for (int k0 = 0; k0 < m0 + 16; k0 += 4) {            // X is lower triangular
            const int kk = k0 + g4;
            const float ax = Xs[(m0 + l16) * PC + kk];
            const float sb = bs[kk], sw = bs[kk] * expf(gcs[kk]);
#pragma unroll
            for (int n = 0; n < NT16; n++) {
                Wt[n] = mfma4(ax, Ks[kk * PD + n * 16 + l16] * sw, Wt[n]);
                Ut[n] = mfma4(ax, Vs[kk * PD + n * 16 + l16] * sb, Ut[n]);
            }
        }
    }
    __syncthreads();
    // stage W (in Qs) and U (in Ks) row-major
#pragma unroll
    for (int n = 0; n < NT16; n++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = wave * 16 + 4 * g4 + r, j = n * 16 + l16;
            Qs[i * PD + j] = Wt[n][r];
            Ks[i * PD + j] = Ut[n][r];
        }
    __syncthreads();
    // 5. W panel (same order as the Q panel) and U panel (D layout per column block)
    for (int e = tid; e < NWV * OMH_WAVE * SS::NFW; e += 256) {
        const int f = e % SS::NFW, l = (e / SS::NFW) % OMH_WAVE, w = e / (SS::NFW * OMH_WAVE);
        const int s = f & 3, kt = (f >> 2) % KT, tt = (f >> 2) / KT;
        const int row = tt * 16 + l % 16, col = 16 * (w * KT + kt) + 4 * (l / 16) + s;
        a.pw[panel_idx((hc * NWV + w) * (SS::NFW / 4), f, l)] = Qs[row * PD + col];
    }
    for (int e = tid; e < NT16 * NWV * OMH_WAVE * SS::NFU; e += 256) {
        // U order per column block cb: f = u*4 + r -> row 16(w*TT+u) + 4g + r, col 16cb + l%16
        const int f = e % SS::NFU, l = (e / SS::NFU) % OMH_WAVE;
        const int w = (e / (SS::NFU * OMH_WAVE)) % NWV, cb = e / (SS::NFU * OMH_WAVE * NWV);
        const int r = f & 3, u = f >> 2;
        const int row = 16 * (w * TT + u) + 4 * (l / 16) + r, col = 16 * cb + l % 16;
        a.pu[panel_idx(((hc * NT16 + cb) * NWV + w) * (SS::NFU / 4), f, l)] = Ks[row * PD + col];
    }
}

// ---------------------------------------------------------------- P3 scan
template <int D>
__global__ __launch_bounds__((ScanShape<D>::NWV * OMH_WAVE), 1)
void prefill_scan_kernel(const PrefillArgs a) {
    using SS = ScanShape<D>;
    constexpr int NWV = SS::NWV, KT = SS::KT, TT = SS::TT;
    constexpr int NCB = D / 16;
    const int vh = a.vh;
    // XCD-aware: the NCB column blocks of a head share one XCD (and its L2)
    int h, cb;
    {
        const int n = blockIdx.x;
        if (vh % 8 == 0) { h = (n % 8) + 8 * (n / (8 * NCB)); cb = (n / 8) % NCB; }
        else { h = n / NCB; cb = n % NCB; }
    }
    const int tid = threadIdx.x, lane = tid % OMH_WAVE, w = tid / OMH_WAVE;
    const int l16 = lane % 16, g4 = lane / 16;

    __shared__ v4f s_p[NWV][4][OMH_WAVE];        // W S partials per wave, token tile
    __shared__ v4f s_o[NWV][4][OMH_WAVE];        // (Q e^gc) S partials
    __shared__ v4f s_vn[4][OMH_WAVE];            // v_new tiles (D layout)

    // S rows 16(w*KT + kt) + 4g + r, column 16cb + l%16
    float *Sbase = a.L.S + ((size_t)a.seq * vh + h) * (D * D);
    v4f S[KT];
#pragma unroll
    for (int kt = 0; kt < KT; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            S[kt][r] = Sbase[(size_t)(16 * (w * KT + kt) + 4 * g4 + r) * D + 16 * cb + l16];

    const size_t vdim = (size_t)vh * D;
    for (int c = 0; c < a.nc; c++) {
        const size_t hc = (size_t)h * a.nc + c;
        float Wf[SS::NFW], Qf[SS::NFW], Kf[SS::NFK], Af[SS::NFA], Uf[SS::NFU];
        {
            const float4 *pw = reinterpret_cast<const float4 *>(a.pw) + (hc * NWV + w) * (SS::NFW / 4) * OMH_WAVE + lane;
            const float4 *pq = reinterpret_cast<const float4 *>(a.pq) + (hc * NWV + w) * (SS::NFW / 4) * OMH_WAVE + lane;
            const float4 *pk = reinterpret_cast<const float4 *>(a.pk) + (hc * NWV + w) * (SS::NFK / 4) * OMH_WAVE + lane;
            const float4 *pa = reinterpret_cast<const float4 *>(a.pa) + (hc * NWV + w) * (SS::NFA / 4) * OMH_WAVE + lane;
            const float4 *pu = reinterpret_cast<const float4 *>(a.pu) + ((hc * NCB + cb) * NWV + w) * (SS::NFU / 4) * OMH_WAVE + lane;
#pragma unroll
            for (int i = 0; i < SS::NFW / 4; i++) {
                const float4 x = pw[i * OMH_WAVE], y = pq[i * OMH_WAVE];
                Wf[4 * i] = x.x; Wf[4 * i + 1] = x.y; Wf[4 * i + 2] = x.z; Wf[4 * i + 3] = x.w;
                Qf[4 * i] = y.x; Qf[4 * i + 1] = y.y; Qf[4 * i + 2] = y.z; Qf[4 * i + 3] = y.w;
            }
#pragma unroll
            for (int i = 0; i < SS::NFK / 4; i++) {
                const float4 x = pk[i * OMH_WAVE];
                Kf[4 * i] = x.x; Kf[4 * i + 1] = x.y; Kf[4 * i + 2] = x.z; Kf[4 * i + 3] = x.w;
            }
#pragma unroll
            for (int i = 0; i < SS::NFA / 4; i++) {
                const float4 x = pa[i * OMH_WAVE];
                Af[4 * i] = x.x; Af[4 * i + 1] = x.y; Af[4 * i + 2] = x.z; Af[4 * i + 3] = x.w;
            }
#pragma unroll
            for (int i = 0; i < SS::NFU / 4; i++) {
                const float4 x = pu[i * OMH_WAVE];
                Uf[4 * i] = x.x; Uf[4 * i + 1] = x.y; Uf[4 * i + 2] = x.z; Uf[4 * i + 3] = x.w;
            }
        }
        const float eg = a.glast[hc];

        // partial W S and (Q e^gc) S over this wave's kd rows, all token tiles
        v4f P[4], O[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            P[tt] = v4zero(); O[tt] = v4zero();
#pragma unroll
            for (int kt = 0; kt < KT; kt++)
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    P[tt] = mfma4(Wf[(tt * KT + kt) * 4 + s], S[kt][s], P[tt]);
                    O[tt] = mfma4(Qf[(tt * KT + kt) * 4 + s], S[kt][s], O[tt]);
                }
            s_p[w][tt][lane] = P[tt];
            s_o[w][tt][lane] = O[tt];
        }
        __syncthreads();
        // reduce over waves for the owned token tiles; v_new = U - W S
        v4f Oa[TT];
#pragma unroll
        for (int u = 0; u < TT; u++) {
            const int mt = w * TT + u;
            v4f p = s_p[0][mt][lane], o = s_o[0][mt][lane];
#pragma unroll
            for (int ww = 1; ww < NWV; ww++) { p += s_p[ww][mt][lane]; o += s_o[ww][mt][lane]; }
            v4f vn;
#pragma unroll
            for (int r = 0; r < 4; r++) vn[r] = Uf[u * 4 + r] - p[r];
            s_vn[mt][lane] = vn;
            Oa[u] = o;
        }
        __syncthreads();
        v4f VN[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) VN[tt] = s_vn[tt][lane];
        // o += Aqk v_new (causal: key tiles <= query tile)
#pragma unroll
        for (int u = 0; u < TT; u++) {
            const int mt = w * TT + u;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
                if (kt <= mt)
#pragma unroll
                    for (int s = 0; s < 4; s++) Oa[u] = mfma4(Af[u * 16 + kt * 4 + s], VN[kt][s], Oa[u]);
            // raw output rows 16mt + 4g + r of this chunk
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = c * C + 16 * mt + 4 * g4 + r;
                if (t < a.T) a.core[(size_t)t * vdim + (size_t)h * D + 16 * cb + l16] = Oa[u][r];
            }
        }
        // S <- e^{gl} S + (K e^{gl-gc})^T v_new
#pragma unroll
        for (int kt = 0; kt < KT; kt++) {
            S[kt] *= eg;
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int s = 0; s < 4; s++) S[kt] = mfma4(Kf[(kt * 4 + tt) * 4 + s], VN[tt][s], S[kt]);
        }
    }
#pragma unroll
    for (int kt = 0; kt < KT; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            Sbase[(size_t)(16 * (w * KT + kt) + 4 * g4 + r) * D + 16 * cb + l16] = S[kt][r];
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <int D>
hipError_t launch_prefill_d(const PrefillArgs &a, hipStream_t st) {
    const int conv_dim = 2 * a.kh * D + a.vh * D;
    hipLaunchKernelGGL((prefill_prep_kernel<D>), dim3(2 * a.kh + a.vh, a.nc), dim3(D < 64 ? 64 : D), 0, st, a);
    hipLaunchKernelGGL(prefill_conv_commit_kernel, dim3((conv_dim + 255) / 256), dim3(256), 0, st, a, conv_dim);
    const size_t lds = (size_t)(3 * C * (D + 4) + 2 * C * (C + 4) + 2 * C) * sizeof(float);
    hipLaunchKernelGGL((prefill_chunk_kernel<D>), dim3(a.vh, a.nc), dim3(256), lds, st, a);
    hipLaunchKernelGGL((prefill_scan_kernel<D>), dim3(a.vh * (D / 16)), dim3(ScanShape<D>::NWV * OMH_WAVE), 0, st, a);
    constexpr int RPB = 256 / (D / 4);
    const size_t rows = (size_t)a.T * a.vh;
    hipLaunchKernelGGL((prefill_gated_norm_kernel<D>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int D>
bool set_lds_limit() {
    const size_t lds = (size_t)(3 * C * (D + 4) + 2 * C * (C + 4) + 2 * C) * sizeof(float);
    return hipFuncSetAttribute((const void *)prefill_chunk_kernel<D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds) == hipSuccess;
}

}  // namespace

size_t prefill_scratch_bytes(int D, int kh, int vh, int T) {
    const size_t Tp = (size_t)((T + C - 1) / C) * C, nc = Tp / C;
    size_t n = 0;
    n += 2 * align256((size_t)kh * Tp * D * 4);            // qn, kn
    n += align256((size_t)vh * Tp * D * 4);                // v
    n += 2 * align256((size_t)vh * Tp * 4);                // g, beta
    n += align256((size_t)vh * Tp * 4);                    // gc (reserved)
    n += align256((size_t)vh * nc * 4);                    // glast
    n += 3 * align256((size_t)vh * Tp * D * 4);            // pw, pq, pk
    n += align256((size_t)vh * nc * C * C * 4);            // pa
    n += align256((size_t)vh * Tp * D * 4);                // pu
    return n;
}

void prefill_bind_scratch(PrefillArgs &a, int D, void *base) {
    const size_t Tp = (size_t)a.Tp, nc = (size_t)a.nc;
    char *p = static_cast<char *>(base);
    auto take = [&](size_t bytes) { float *r = reinterpret_cast<float *>(p); p += align256(bytes); return r; };
    a.qn = take((size_t)a.kh * Tp * D * 4);
    a.kn = take((size_t)a.kh * Tp * D * 4);
    a.v = take((size_t)a.vh * Tp * D * 4);
    a.g = take((size_t)a.vh * Tp * 4);
    a.beta = take((size_t)a.vh * Tp * 4);
    a.gc = take((size_t)a.vh * Tp * 4);
    a.glast = take((size_t)a.vh * nc * 4);
    a.pw = take((size_t)a.vh * Tp * D * 4);
    a.pq = take((size_t)a.vh * Tp * D * 4);
    a.pk = take((size_t)a.vh * Tp * D * 4);
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
