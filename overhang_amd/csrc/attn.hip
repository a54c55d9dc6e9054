// attn.hip — the gated full-attention layer of the Qwen3.5/3.6 engine
// (engines/qwen.c:366-425, attn_step), the layer that every fourth block runs
// beside the GDN layers, for T new tokens of one sequence at positions
// pos .. pos+T-1.
//
// After the qkv projection (one launch_proj over the concatenated rows
// [H x (q | gate), KV x k, KV x v], qwen.c:370-374) three launches:
//  1. attn_prep_kernel, one workgroup per token (its RoPE cos / sin computed
//     once, then a wave per head row; decode steps do this inside the split
//     kernel instead): RMSNorm of q and k with
//     (1 + w) weights (qwen.c:148-152, 385-386), partial RoPE over the first
//     rot dims as two non-interleaved halves (qwen.c:388-398, inverse
//     frequencies computed on the host as there), then q into a scratch row
//     and k, v into the sequence's cache rows pos + t (qwen.c:400-404).
//  2. the split kernel, flash-decoding: one workgroup per (key split, kv
//     head, token) reads the split's K and V rows once for all the query
//     heads of its group (GQA, qwen.c:408-409), keeps a running max and sum
//     per head (online softmax) and writes unnormalised partials.  Head
//     widths of 64 and more: attn_split_mfma_kernel, K and V from HBM
//     straight into fp32 MFMA operands (the heads of the group are the
//     products' 16 columns).  Width 32: attn_split_kernel, 64-key tiles
//     staged through LDS, lane = key for the scores (q broadcast from LDS),
//     lane = 4 output columns for P.V (each key's weight by readlane).
//  3. attn_combine_kernel, per (token, head, 64 columns): merges the splits,
//     normalises, and applies the output gate sigmoid(gate) (qwen.c:421).
// The o_proj is a second launch_proj.
//
// Decode is HBM-bound on the visible cache: 2 * KV * n * hd * 4 bytes for
// n = pos + 1 keys; the splits give >= 256 workgroups (one per CU, as the
// LDS footprint allows).  Token t
// sees keys 0 .. pos+t (causal), and the key tiles beyond that are masked.
#include "omh_internal.h"
#include "omh_device.h"

#include <math.h>

namespace omh {
namespace {

template <int HD>
struct AttnShape {
    static constexpr int KT = 64;                 // keys per tile
    static constexpr int KS = HD + 4;             // padded K row in LDS (floats)
    static constexpr int NG4 = HD / 4;            // float4 groups per row
    static constexpr int R4 = (NG4 + OMH_WAVE - 1) / OMH_WAVE;   // groups per lane in P.V
    static constexpr int NW = 8;                  // waves (two per SIMD)
    static constexpr size_t LDS = (size_t)(kAttnMaxGroup * HD + KT * KS + KT * HD) * sizeof(float);
};

__device__ __forceinline__ float wave_max(float v) { return omh_lane_max(v); }

// cos and sin of p * inv[j] for j < rot / 2 into LDS tables, by the threads
// of a workgroup.  One out-of-line function computes them wherever a kernel
// needs them, so every kernel rotates with the same bits.
__device__ __attribute__((noinline)) void rope_cos_sin(float ang, float *c, float *s) {
    *c = cosf(ang);
    *s = sinf(ang);
}
__device__ __forceinline__ void rope_table(const AttnArgs &a, int p, float *cs, float *sn, int tid, int nthreads) {
    for (int j = tid; j < a.rot / 2; j += nthreads) rope_cos_sin((float)p * a.inv[j], cs + j, sn + j);
}

// One q or k row of the prep (RMSNorm with 1 + w, then partial RoPE as two
// non-interleaved halves), or a v row (no weights: copied), by one wave,
// into an LDS row (the RoPE pairs are read back from it).  cs_t / sn_t: the
// token's rope_table.  prep_row_regs takes the row (v, element lane + 64 i
// in v[i]) and the weights (wv, likewise) already in registers, so a caller
// can issue those loads ahead of others; prep_row loads them itself.  On
// return v holds the row as written (its fences order LDS only, so global
// loads a caller issued ahead stay in flight).
template <int HD>
__device__ __forceinline__ void prep_row_regs(const AttnArgs &a, float (&v)[(HD + OMH_WAVE - 1) / OMH_WAVE],
                                              const float (&wv)[(HD + OMH_WAVE - 1) / OMH_WAVE], bool norm, float *row,
                                              int lane, const float *cs_t, const float *sn_t) {
    constexpr int NE = (HD + OMH_WAVE - 1) / OMH_WAVE;
    if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NE; i++) ss += v[i] * v[i];
        ss = omh_xor_sum_from<1>(ss);
        const float rr = 1.f / sqrtf(ss / (float)HD + a.eps);   // qwen.c:148-152
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < HD) {
                v[i] = v[i] * rr * (1.f + wv[i]);
                row[j] = v[i];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // the wave's row is in LDS
        __builtin_amdgcn_wave_barrier();
        const int half = a.rot / 2;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < a.rot) {                                     // qwen.c:388-398
                const int jj = j < half ? j : j - half;
                const float cs = cs_t[jj], sn = sn_t[jj];
                const float a0 = row[jj], b0 = row[jj + half];
                v[i] = j < half ? a0 * cs - b0 * sn : b0 * cs + a0 * sn;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // every lane has read its pair
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int j = lane + OMH_WAVE * i;
        if (j < HD) row[j] = v[i];
    }
}
template <int HD>
__device__ __forceinline__ void prep_row(const AttnArgs &a, const float *src, const float *w, float *row, int lane,
                                         const float *cs_t, const float *sn_t) {
    constexpr int NE = (HD + OMH_WAVE - 1) / OMH_WAVE;
    float v[NE], wv[NE];
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int j = lane + OMH_WAVE * i;
        v[i] = j < HD ? src[j] : 0.f;
        wv[i] = w && j < HD ? w[j] : 0.f;
    }
    prep_row_regs<HD>(a, v, wv, w != nullptr, row, lane, cs_t, sn_t);
}

// The prep: one workgroup of kPrepWaves waves per token.  The token's RoPE
// cos and sin (rot / 2 frequencies) go into LDS once, then wave w takes rows
// w, w + kPrepWaves, ... of [H q heads, KV k heads, KV v heads]: q into the
// scratch, k and v into the cache rows pos + t.  A wave's next row (and its
// norm weights) is requested before the current one is formed, and its
// first before the RoPE table, so the rows' HBM round trips overlap.
constexpr int kPrepWaves = 4;
template <int HD>
__global__ __launch_bounds__(kPrepWaves * OMH_WAVE) void attn_prep_kernel(const AttnArgs a) {
    constexpr int NE = (HD + OMH_WAVE - 1) / OMH_WAVE;
    __shared__ float cs[HD / 2], sn[HD / 2], sv[kPrepWaves][HD];
    const int H = a.H, KV = a.KV, nr = H + 2 * KV;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int p = a.pos + t;
    const float *row = a.qkv + (size_t)t * a.ld_qkv;
    // row r's source and norm weights (null: a v row, copied)
    auto src_of = [&](int r, const float *&w) -> const float * {
        if (r < H) { w = a.qn; return row + (size_t)r * 2 * HD; }                          // q of head r (then its gate)
        if (r < H + KV) { w = a.kn; return row + (size_t)2 * H * HD + (size_t)(r - H) * HD; }   // k of kv head r - H
        w = nullptr;
        return row + (size_t)2 * H * HD + (size_t)(r - H) * HD;                          // v of kv head r - H - KV
    };
    float v[NE], wt[NE];
    auto fetch = [&](int r) __attribute__((always_inline)) {
        const float *w;
        const float *src = src_of(r, w);
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            v[i] = j < HD ? src[j] : 0.f;
            wt[i] = w && j < HD ? w[j] : 0.f;
        }
    };
    if (wv < nr) fetch(wv);
    rope_table(a, p, cs, sn, tid, kPrepWaves * OMH_WAVE);
    __syncthreads();
    for (int r = wv; r < nr; r += kPrepWaves) {
        float cv[NE], cw[NE];
#pragma unroll
        for (int i = 0; i < NE; i++) {
            cv[i] = v[i];
            cw[i] = wt[i];
        }
        if (r + kPrepWaves < nr) fetch(r + kPrepWaves);
        float *dst;
        if (r < H) dst = a.qb + ((size_t)t * H + r) * HD;
        else if (r < H + KV) dst = a.Kc + (((size_t)a.seq * KV + (r - H)) * a.max_t + p) * HD;
        else dst = a.Vc + (((size_t)a.seq * KV + (r - H - KV)) * a.max_t + p) * HD;
        prep_row_regs<HD>(a, cv, cw, r < H + KV, sv[wv], lane, cs, sn);
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < HD) dst[j] = cv[i];
        }
    }
}


// GPW = query heads per wave (the group's heads grp spread over the NW
// waves: head wave + NW*i).  The hot loops carry no per-head conditions (a
// branch there serialises every LDS read behind its own wait): a wave
// whose head index runs past grp computes a copy of head grp-1 and does not
// write it.
// PREP (decode steps, T = 1): the prep kernel's work is done here instead
// of in a launch of its own: every workgroup forms its group's q rows
// straight into LDS, and the workgroup whose split holds position pos writes
// the new k and v rows into the cache before it reads any tile.
template <int HD, int GPW, bool PREP = false>
__global__ __launch_bounds__(AttnShape<HD>::NW * OMH_WAVE) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_split_kernel(const AttnArgs a) {   // one workgroup per CU (LDS): all of each SIMD's registers
    using S = AttnShape<HD>;
    constexpr int R4 = S::R4, NG4 = S::NG4, KT = S::KT, NW = S::NW, NT = NW * OMH_WAVE;
    extern __shared__ float smem[];
    float *qs = smem;                              // [group heads][HD]
    float *Ks = qs + kAttnMaxGroup * HD;           // [KT][KS]
    float *Vs = Ks + KT * S::KS;                   // [KT][HD]

    const int H = a.H, KV = a.KV, grp = H / KV, ns = a.ns;
    const int s = blockIdx.x % ns, g = (blockIdx.x / ns) % KV, t = blockIdx.x / (ns * KV);
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int n = a.pos + t + 1;                   // keys token t sees
    const int k0 = s * a.kps, k1 = min(n, k0 + a.kps);
    // partial of query head g*grp + i: index pb + i*ns
    const size_t pb = ((size_t)t * H + (size_t)g * grp) * ns + s;
    if (k0 >= k1) {                                // an empty split: weight zero in the merge
        for (int e = tid; e < grp * NG4; e += NT) {
            const size_t pi = pb + (size_t)(e / NG4) * ns;
            *reinterpret_cast<float4 *>(a.po + pi * HD + 4 * (e % NG4)) = f4_zero();
            if (e % NG4 == 0) {
                a.pml[2 * pi] = -INFINITY;
                a.pml[2 * pi + 1] = 0.f;
            }
        }
        return;
    }
    if constexpr (PREP) {
        const int p = a.pos + t;
        const float *row = a.qkv + (size_t)t * a.ld_qkv;
        float *cs = Ks + HD, *sn = cs + HD / 2;     // (the K tile region is free until the first tile)
        rope_table(a, p, cs, sn, tid, NT);
        __syncthreads();
        if (k0 <= p && p < k1) {
            // the new k (wave 0, normed and rotated through a scratch LDS row)
            // and v (wave 1) of kv head g go into the cache rows p
            const size_t crow = (((size_t)a.seq * KV + g) * a.max_t + p) * HD;
            if (wave == 0) {
                prep_row<HD>(a, row + (size_t)2 * H * HD + (size_t)g * HD, a.kn, Ks, lane, cs, sn);
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
                __builtin_amdgcn_wave_barrier();
                for (int j = lane; j < HD; j += OMH_WAVE) a.Kc[crow + j] = Ks[j];
            } else if (wave == 1) {
                for (int j = lane; j < HD; j += OMH_WAVE) a.Vc[crow + j] = row[(size_t)2 * H * HD + (size_t)(KV + g) * HD + j];
            }
            __threadfence();                       // the rows are in memory before any tile load reads them
            __syncthreads();
        }
        for (int i = wave; i < grp; i += NW)
            prep_row<HD>(a, row + (size_t)(g * grp + i) * 2 * HD, a.qn, qs + i * HD, lane, cs, sn);
    } else {
        for (int e = tid; e < grp * NG4; e += NT) {
            const int i = e / NG4, c = e % NG4;
            *reinterpret_cast<float4 *>(qs + i * HD + 4 * c) =
                *reinterpret_cast<const float4 *>(a.qb + ((size_t)t * H + (size_t)g * grp + i) * HD + 4 * c);
        }
    }
    const float *qh[GPW];                          // this wave's heads' q rows in LDS
#pragma unroll
    for (int i = 0; i < GPW; i++) qh[i] = qs + min(wave + NW * i, grp - 1) * HD;
    float m[GPW], l[GPW];
    float4 o[GPW][R4];
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        m[i] = -INFINITY;
        l[i] = 0.f;
#pragma unroll
        for (int r = 0; r < R4; r++) o[i][r] = f4_zero();
    }
    const size_t cache0 = ((size_t)a.seq * KV + g) * a.max_t;
    const float *Kg = a.Kc + cache0 * HD, *Vg = a.Vc + cache0 * HD;

    // K and V tiles go HBM -> registers -> LDS: every thread's PER pieces of
    // a tile are in flight at once, and the next tile's loads are issued as
    // soon as the current one is in LDS, so they overlap its compute.  Rows
    // past the split's end repeat the tile's first row, so every LDS row
    // holds finite values (their weights are zero).
    constexpr int PER = KT * NG4 / NT;
    static_assert(KT * NG4 % NT == 0, "tile pieces per thread");
    omh_v4f kr[PER], vr[PER];                      // native vectors: HIP's float4 copies stay in scratch
#define OMH_ATTN_LOAD_PIECE(I, KT0, NK)                                                   \
    {                                                                                     \
        const int e = tid + NT * (I), kk = e / NG4, c = e % NG4;                          \
        const size_t off = (size_t)((KT0) + (kk < (NK) ? kk : 0)) * HD + 4 * c;           \
        kr[I] = *reinterpret_cast<const omh_v4f *>(Kg + off);                             \
        vr[I] = *reinterpret_cast<const omh_v4f *>(Vg + off);                             \
    }
#pragma unroll
    for (int i = 0; i < PER; i++) OMH_ATTN_LOAD_PIECE(i, k0, min(KT, k1 - k0))
    for (int kt = k0; kt < k1; kt += KT) {
        const int nk = min(KT, k1 - kt);
        omh_lds_barrier();                         // the previous tile's readers are done
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int e = tid + NT * i, kk = e / NG4, c = e % NG4;
            *reinterpret_cast<omh_v4f *>(Ks + kk * S::KS + 4 * c) = kr[i];
            *reinterpret_cast<omh_v4f *>(Vs + kk * HD + 4 * c) = vr[i];
        }
        omh_lds_barrier();
        // the next tile's pieces are issued spread over the score blocks
        // below; after the last tile they re-read this one (cache hits)
        const bool more = kt + KT < k1;
        const int kn = more ? kt + KT : kt, nkn = more ? min(KT, k1 - kt - KT) : nk;

        // scores q.k * hd^-1/2 (qwen.c:410-414), lane = key
        const bool valid = lane < nk;
        const float *kr_l = Ks + lane * S::KS;
        float acc[GPW], pl[GPW];
#pragma unroll
        for (int i = 0; i < GPW; i++) acc[i] = 0.f;
        constexpr int CB = 8, NB = NG4 / CB, PPB = (PER + NB - 1) / NB;
        static_assert(NG4 % CB == 0, "score blocks");
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int u = 0; u < PPB; u++)
                if (b * PPB + u < PER) OMH_ATTN_LOAD_PIECE(b * PPB + u, kn, nkn)
#pragma unroll
            for (int cc = 0; cc < CB; cc++) {
                const int c = b * CB + cc;
                const float4 kv = *reinterpret_cast<const float4 *>(kr_l + 4 * c);
#pragma unroll
                for (int i = 0; i < GPW; i++) {
                    const float4 q = *reinterpret_cast<const float4 *>(qh[i] + 4 * c);
                    acc[i] = fmaf(q.x, kv.x, acc[i]);
                    acc[i] = fmaf(q.y, kv.y, acc[i]);
                    acc[i] = fmaf(q.z, kv.z, acc[i]);
                    acc[i] = fmaf(q.w, kv.w, acc[i]);
                }
            }
        }
        // online softmax (qwen.c:413 softmax_ over all keys, merged per tile)
#pragma unroll
        for (int i = 0; i < GPW; i++) {
            const float sc = valid ? acc[i] * a.scale : -INFINITY;
            const float mn = fmaxf(m[i], wave_max(sc));
            const float corr = expf(m[i] - mn);
            const float pe = valid ? expf(sc - mn) : 0.f;
            l[i] = l[i] * corr + omh_xor_sum_from<1>(pe);
#pragma unroll
            for (int r = 0; r < R4; r++) o[i][r] = f4_scale(o[i][r], corr);
            pl[i] = pe;
            m[i] = mn;
        }

        // P.V (qwen.c:415-419), lane = 4 columns; the weight of key kk is
        // lane kk's pl (zero past nk), broadcast by readlane
#pragma unroll 8
        for (int kk = 0; kk < KT; kk++) {
            float4 vv[R4];
#pragma unroll
            for (int r = 0; r < R4; r++) {
                const int c = min(lane + OMH_WAVE * r, NG4 - 1);
                vv[r] = *reinterpret_cast<const float4 *>(Vs + kk * HD + 4 * c);
            }
#pragma unroll
            for (int i = 0; i < GPW; i++) {
                const float pv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pl[i]), kk));
#pragma unroll
                for (int r = 0; r < R4; r++) o[i][r] = f4_fma(vv[r], pv, o[i][r]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        const int h = wave + NW * i;
        if (h < grp) {
            const size_t pi = pb + (size_t)h * ns;
#pragma unroll
            for (int r = 0; r < R4; r++) {
                const int c = lane + OMH_WAVE * r;
                if (c < NG4) *reinterpret_cast<float4 *>(a.po + pi * HD + 4 * c) = o[i][r];
            }
            if (lane == 0) {
                a.pml[2 * pi] = m[i];
                a.pml[2 * pi + 1] = l[i];
            }
        }
    }
}
#undef OMH_ATTN_LOAD_PIECE

// ---------------------------------------------------------------- decode on the matrix cores
// The split kernel for head widths of 64 and more: the same work unit (one
// key split of one kv head for one token, the prep folded in for decode
// steps), with K and V going from HBM straight into fp32 MFMA operands, so
// every key row is read once for all the group's query heads (no LDS
// staging, no per-head re-reads).  Each of the NW waves streams its own
// 16-key blocks (blocks w, w + NW, ...) and keeps its own online softmax.
// A wave holds one operand set: a block's K rows, then (once the scores are
// formed) its V rows in the same registers; the two waves of a SIMD overlap
// one's loads with the other's products:
//   S^T = K Q^T   (v_mfma_f32_16x16x4_f32; A = K rows, lane l16 = key;
//                  B = q from LDS, lane l16 = query head of the group, heads
//                  past the group zero; head dims taken in the order 16 i + 4 g + s
//                  on both operands, one 16-byte K load per 4 products),
//   O += P V      (A = the probabilities as the score product left them:
//                  key 4 g + s of lane group g is register s; B = V rows
//                  4 g + s, lane l16 = output columns 64 q + 4 l16 + c of
//                  tile 4 q + c, so one 16-byte V load serves 4 tiles).
// The waves' (max, sum, O) then merge through LDS into the split's partial,
// which the combine kernel merges with the other splits as before.  Keys
// past the split's end or the token's position are masked (their rows
// repeat a visible row, so every operand is finite).
template <int HD>
struct MfmaSplitShape {
    static constexpr int NW = 8;                   // waves, two per SIMD
    static constexpr int QS = HD + 4;              // padded q row in LDS
    static constexpr int NI = HD / 16;             // K float4s per lane per block (4 k-steps each)
    static constexpr int NQ = HD / 64;             // V float4s per lane per key step
    static constexpr size_t LDS = (size_t)(kAttnMaxGroup * QS + NW * 16 * HD + 2 * NW * 16) * sizeof(float);
    static_assert(HD % 64 == 0, "64-column V groups");
};

__device__ __forceinline__ omh_v4f ld_stream_v4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(omh_v4f, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kOmhNT));
}

template <int HD, bool PREP>
__global__ __launch_bounds__(MfmaSplitShape<HD>::NW * OMH_WAVE, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_split_mfma_kernel(const AttnArgs a) {
    using S = MfmaSplitShape<HD>;
    constexpr int NW = S::NW, NT = NW * OMH_WAVE, QS = S::QS, NI = S::NI, NQ = S::NQ;
    extern __shared__ float smem[];
    float *qs = smem;                              // [kAttnMaxGroup][QS] the group's q rows
    float *mo = qs + kAttnMaxGroup * QS;           // [NW][16][HD] the waves' outputs (the prep's scratch before)
    float *mm = mo + NW * 16 * HD;                 // [NW][16] running max, then [NW][16] sums

    const int H = a.H, KV = a.KV, grp = H / KV, ns = a.ns;
    const int s = blockIdx.x % ns, g = (blockIdx.x / ns) % KV, t = blockIdx.x / (ns * KV);
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, g4 = lane / 16;
    const int n = a.pos + t + 1;                   // keys token t sees
    const int k0 = s * a.kps, k1 = min(n, k0 + a.kps);
    const size_t pb = ((size_t)t * H + (size_t)g * grp) * ns + s;
    if (k0 >= k1) {                                // an empty split: weight zero in the merge
        for (int e = tid; e < grp * (HD / 4); e += NT) {
            const size_t pi = pb + (size_t)(e / (HD / 4)) * ns;
            *reinterpret_cast<float4 *>(a.po + pi * HD + 4 * (e % (HD / 4))) = f4_zero();
            if (e % (HD / 4) == 0) {
                a.pml[2 * pi] = -INFINITY;
                a.pml[2 * pi + 1] = 0.f;
            }
        }
        return;
    }
    const size_t cache0 = ((size_t)a.seq * KV + g) * a.max_t * HD;
    const int cbytes = a.max_t * HD * (int)sizeof(float);          // (launch_attn_d checks the range)
    const __amdgpu_buffer_rsrc_t krs = omh_rsrc(a.Kc + cache0, cbytes), vrs = omh_rsrc(a.Vc + cache0, cbytes);
    const int nb = (k1 - k0 + 15) / 16;            // 16-key blocks of the split
    // one operand set: a block's K rows (lane (l16, g4): key l16, dims
    // 16 i + 4 g4 .. +3 in kv[i]), then its V rows (key 4 g4 + st, columns
    // 64 q + 4 l16 .. +3 in kv[NQ st + q])
    static_assert(NI == 4 * NQ, "K and V fill the same registers");
    omh_v4f kv[NI];
    auto load_k = [&](int b) __attribute__((always_inline)) {
        const int kk = min(k0 + 16 * b + l16, k1 - 1);
#pragma unroll
        for (int i = 0; i < NI; i++) kv[i] = ld_stream_v4(krs, (kk * HD + 16 * i + 4 * g4) * 4);
    };
    auto load_v = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int kr = min(k0 + 16 * b + 4 * g4 + st, k1 - 1);
#pragma unroll
            for (int q = 0; q < NQ; q++) kv[NQ * st + q] = ld_stream_v4(vrs, (kr * HD + 64 * q + 4 * l16) * 4);
        }
    };
    // Prologue.  A decode step's RoPE table comes first (its out-of-line
    // cos / sin call waits for every load the wave has in flight), and the
    // split holding the step's position writes the new k / v cache rows.
    // Then the loads the q prep needs (the group's q rows, the norm weights)
    // and the first K / V block of the wave go out, in that order, in
    // straight-line code: loads complete in issue order, so the prep's waits
    // leave the block's loads in flight.  A prompt step's prepared q rows go
    // to LDS before the block loads.
    const int p = a.pos + t;
    if constexpr (PREP) {
        const float *row = a.qkv + (size_t)t * a.ld_qkv;
        float *krow = mo, *cs = mo + HD, *sn = cs + HD / 2;
        rope_table(a, p, cs, sn, tid, NT);
        __syncthreads();
        if (k0 <= p && p < k1) {
            // the new k (wave 0, normed and rotated through a scratch LDS row)
            // and v (wave 1) of kv head g go into the cache rows p
            const size_t crow = (((size_t)a.seq * KV + g) * a.max_t + p) * HD;
            if (wave == 0) {
                prep_row<HD>(a, row + (size_t)2 * H * HD + (size_t)g * HD, a.kn, krow, lane, cs, sn);
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
                __builtin_amdgcn_wave_barrier();
                for (int j = lane; j < HD; j += OMH_WAVE) a.Kc[crow + j] = krow[j];
            } else if (wave == 1) {
                for (int j = lane; j < HD; j += OMH_WAVE) a.Vc[crow + j] = row[(size_t)2 * H * HD + (size_t)(KV + g) * HD + j];
            }
            __threadfence();                       // the rows are in memory before any block load reads them
            __syncthreads();
        }
        constexpr int NE = HD / OMH_WAVE, MAXH = (kAttnMaxGroup + NW - 1) / NW;
        float xv[MAXH][NE], wn[NE];
#pragma unroll
        for (int k = 0; k < MAXH; k++) {
            const int i = min(wave + NW * k, grp - 1);
#pragma unroll
            for (int e = 0; e < NE; e++) xv[k][e] = row[(size_t)(g * grp + i) * 2 * HD + lane + OMH_WAVE * e];
        }
#pragma unroll
        for (int e = 0; e < NE; e++) wn[e] = a.qn[lane + OMH_WAVE * e];
#pragma unroll
        for (int k = 0; k < MAXH; k++) {
            const int i = wave + NW * k;
            if (i < grp) prep_row_regs<HD>(a, xv[k], wn, true, qs + i * QS, lane, cs, sn);
        }
        load_k(wave);
    } else {
        for (int e = tid; e < grp * (HD / 4); e += NT) {
            const int i = e / (HD / 4), c = e % (HD / 4);
            *reinterpret_cast<float4 *>(qs + i * QS + 4 * c) =
                *reinterpret_cast<const float4 *>(a.qb + ((size_t)t * H + (size_t)g * grp + i) * HD + 4 * c);
        }
        load_k(wave);
    }
    // (LDS-only barriers from here on: a full __syncthreads would also wait
    // for the block loads in flight)
    omh_lds_barrier();
    // q as the B operand: lane (g4, head l16) reads q[l16][16 i + 4 g4 .. +3]
    // (rows past the group read as zero)
    if (grp < 16) {
        for (int e = tid; e < (16 - grp) * (HD / 4); e += NT)
            *reinterpret_cast<float4 *>(qs + (grp + e / (HD / 4)) * QS + 4 * (e % (HD / 4))) = f4_zero();
        omh_lds_barrier();
    }
    const float *qrow = qs + l16 * QS + 4 * g4;

    float m = -INFINITY, l = 0.f;                  // of head l16 (the same in the four lane groups)
    omh_v4f o[NI];                                 // O rows 4 g4 + r, columns 64 q + 4 l16 + c of tile 4 q + c
#pragma unroll
    for (int dt = 0; dt < NI; dt++) o[dt] = omh_v4f{0.f, 0.f, 0.f, 0.f};

    auto step = [&](int b) __attribute__((always_inline)) {
        // scores of keys kb + 4 g4 + r for head l16 (two product chains)
        omh_v4f sa = omh_v4f{0.f, 0.f, 0.f, 0.f}, sb = sa;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const omh_v4f qf = *reinterpret_cast<const omh_v4f *>(qrow + 16 * i);
#pragma unroll
            for (int st = 0; st < 4; st++) {
                if (i & 1) sb = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i][st], qf[st], sb, 0, 0, 0);
                else sa = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i][st], qf[st], sa, 0, 0, 0);
            }
        }
        load_v(b);                                 // (into the registers the scores have read)
        const int kb = k0 + 16 * b;
        float sc[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[r] = kb + 4 * g4 + r < k1 ? (sa[r] + sb[r]) * a.scale : -INFINITY;   // qwen.c:410-414
            mx = fmaxf(mx, sc[r]);
        }
        mx = omh_swap32_max(omh_swap16_max(mx));
        // online softmax (qwen.c:413 softmax_ over all keys, merged per block);
        // the block's first key is visible, so mn is finite
        const float mn = fmaxf(m, mx);
        const float corr = expf(m - mn);
        float pr[4], ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            pr[r] = kb + 4 * g4 + r < k1 ? expf(sc[r] - mn) : 0.f;
            ps += pr[r];
        }
        ps = omh_swap32_sum(omh_swap16_sum(ps));
        l = l * corr + ps;
        m = mn;
        // the output rows are heads 4 g4 + r: their corrections from lanes 4 g4 + r
        float cr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) cr[r] = __shfl(corr, 4 * g4 + r, OMH_WAVE);
#pragma unroll
        for (int dt = 0; dt < NI; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] *= cr[r];
        // P.V (qwen.c:415-419)
#pragma unroll
        for (int q = 0; q < NQ; q++)
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int st = 0; st < 4; st++)
                    o[4 * q + c] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[st], kv[NQ * st + q][c], o[4 * q + c], 0, 0, 0);
    };
    // the wave's blocks wave, wave + NW, ... (block wave's loads went out above)
    for (int b = wave; b < nb; b += NW) {
        if (b != wave) load_k(b);
        step(b);
    }

    // merge the waves: the workgroup's max per head, each wave's output scaled to it
    if (g4 == 0) {
        mm[wave * 16 + l16] = m;
        mm[NW * 16 + wave * 16 + l16] = l;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int h = 4 * g4 + r;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, mm[w * 16 + h]);
        const float f = expf(mm[wave * 16 + h] - M);        // 0 for a wave without blocks (its m is -inf)
#pragma unroll
        for (int q = 0; q < NQ; q++)
            *reinterpret_cast<omh_v4f *>(mo + (wave * 16 + h) * HD + 64 * q + 4 * l16) =
                omh_v4f{o[4 * q][r] * f, o[4 * q + 1][r] * f, o[4 * q + 2][r] * f, o[4 * q + 3][r] * f};
    }
    __syncthreads();
    for (int e = tid; e < grp * (HD / 4); e += NT) {
        const int i = e / (HD / 4), c = e % (HD / 4);
        omh_v4f acc = *reinterpret_cast<const omh_v4f *>(mo + i * HD + 4 * c);
#pragma unroll
        for (int w = 1; w < NW; w++) acc += *reinterpret_cast<const omh_v4f *>(mo + (w * 16 + i) * HD + 4 * c);
        *reinterpret_cast<omh_v4f *>(a.po + (pb + (size_t)i * ns) * HD + 4 * c) = acc;
    }
    if (tid < grp) {
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, mm[w * 16 + tid]);
#pragma unroll
        for (int w = 0; w < NW; w++) L += mm[NW * 16 + w * 16 + tid] * expf(mm[w * 16 + tid] - M);
        const size_t pi = pb + (size_t)tid * ns;
        a.pml[2 * pi] = M;
        a.pml[2 * pi + 1] = L;
    }
}

// ---------------------------------------------------------------- prompt steps
// Flash attention on the matrix cores for prompt steps of at least
// kFlashMinT tokens (attn_flash3_kernel below: bf16 x 3 products, the
// default; this one with fp32 products, v_mfma_f32_16x16x4f32, kept for
// comparison, OMH_ATTN_FLASH=fp32): the same fp32 scores, online
// softmax and P.V as the split kernel, as dense products.  A wave owns one
// unit, 16 consecutive tokens of one query head; a workgroup of 8 waves
// takes 8 units of one kv group (the group's heads of a token block, then
// the next block), so the K and V tiles it stages in LDS (32 keys, double
// buffered, HBM -> registers -> LDS one tile ahead) serve 8 waves.  Per
// wave, S^T = K Q^T (A = a K row from LDS, B = the wave's q, held in
// registers for the whole sweep), so each lane's scores belong to its own
// query row (lane % 16): the row max and sum need two exchanges and the
// rescale of the output is lane-local; O^T = V^T P^T (A = V from LDS, B =
// the probabilities as the score product left them: key 16 n + 4 g + s of
// lane group g is register s).  The head dims of q.k are taken in the order
// 16 c + 4 g + s on both operands (one 16-byte K read per 4 products).  The
// workgroups holding the most keys (the prompt's end) start first.  Keys
// past a token's position are masked; rows of the last tile past the
// visible keys repeat the tile's first row, so every LDS value is finite.
template <int HD>
struct FlashShape {
    static constexpr int KT = 32;                  // keys per tile
    static constexpr int LD = HD + 4;              // padded row in LDS (floats)
    static constexpr int STAGE = 2 * KT * LD;      // one stage: K rows, then V rows
    static constexpr size_t LDS = 2 * (size_t)STAGE * sizeof(float);
    static constexpr int NC = HD / 16;             // 16-dim groups (q registers; output tiles)
    static constexpr int PER = KT * HD / 4 / (8 * OMH_WAVE);   // float4 pieces of K (and of V) per thread
};
constexpr int kFlashMinT = 64;
// decode steps fold the prep into the split kernel unless OMH_ATTN_FUSE=0 (comparison)
bool fuse_prep() {
    const char *e = getenv("OMH_ATTN_FUSE");
    return !(e && e[0] == '0');
}
// the fp32-product flash kernel instead of the bf16 x 3 one (OMH_ATTN_FLASH=fp32, for comparison)
bool flash_fp32() {
    const char *e = getenv("OMH_ATTN_FLASH");
    return e && e[0] == 'f';
}
// the bf16 x 3 kernel converting every tile itself instead of copying tile
// images (OMH_ATTN_FLASH=reg, for comparison)
bool flash_reg() {
    const char *e = getenv("OMH_ATTN_FLASH");
    return e && e[0] == 'r';
}
// prompt steps of at least this many tokens stage their tiles from images
constexpr int kFlashImageMinT = 256;

template <int HD>
__global__ __launch_bounds__(8 * OMH_WAVE) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_flash_kernel(const AttnArgs a) {
    using F = FlashShape<HD>;
    constexpr int KT = F::KT, LD = F::LD, NC = F::NC, PER = F::PER, NT = 8 * OMH_WAVE;
    extern __shared__ float smem[];
    const int H = a.H, KV = a.KV, grp = H / KV;
    const int nunit = (a.T + 15) / 16 * grp, wpg = (nunit + 7) / 8;
    const int g = blockIdx.x % KV, wi = wpg - 1 - (int)blockIdx.x / KV;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, gq = lane / 16;
    const bool own = 8 * wi + w < nunit;
    const int u = min(8 * wi + w, nunit - 1);
    const int tb = u / grp, h = g * grp + u % grp;
    const int tq = 16 * tb + l16;                  // this lane's query token (may be past T: not written)
    const int tlast = min(16 * (min(8 * wi + 7, nunit - 1) / grp) + 15, a.T - 1);
    const int nkeys = a.pos + tlast + 1;           // keys the workgroup's last token sees
    const int kmax = a.pos + tq;                   // the last key this lane's token sees

    omh_v4f q[NC];                                 // dims 16 c + 4 gq .. +3 of token tq
    {
        const float *qr = a.qb + ((size_t)min(tq, a.T - 1) * H + h) * HD + 4 * gq;
#pragma unroll
        for (int c = 0; c < NC; c++) q[c] = *reinterpret_cast<const omh_v4f *>(qr + 16 * c);
    }
    const size_t cache0 = ((size_t)a.seq * KV + g) * a.max_t;
    const float *Kg = a.Kc + cache0 * HD, *Vg = a.Vc + cache0 * HD;
    omh_v4f kr[PER], vr[PER];
    auto load = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int e = tid + NT * i, kk = e / (HD / 4), c = e % (HD / 4);
            const size_t off = (size_t)(kt + kk < nkeys ? kt + kk : kt) * HD + 4 * c;
            kr[i] = *reinterpret_cast<const omh_v4f *>(Kg + off);
            vr[i] = *reinterpret_cast<const omh_v4f *>(Vg + off);
        }
    };
    auto put = [&](int stage) __attribute__((always_inline)) {
        float *Ks = smem + stage * F::STAGE, *Vs = Ks + KT * LD;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int e = tid + NT * i, kk = e / (HD / 4), c = e % (HD / 4);
            *reinterpret_cast<omh_v4f *>(Ks + kk * LD + 4 * c) = kr[i];
            *reinterpret_cast<omh_v4f *>(Vs + kk * LD + 4 * c) = vr[i];
        }
    };

    omh_v4f o[NC];                                     // O^T: o[j][i] = O[token tq][dim 16 j + 4 gq + i]
#pragma unroll
    for (int j = 0; j < NC; j++) o[j] = omh_v4f{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    load(0);
    put(0);
    __syncthreads();
    for (int kt = 0, st = 0; kt < nkeys; kt += KT, st ^= 1) {
        if (kt + KT < nkeys) load(kt + KT);
        const float *Ks = smem + st * F::STAGE, *Vs = Ks + KT * LD;
        // S^T for keys kt + 16 n + 4 gq + i (register i of sc[n]), query row tq
        omh_v4f sc[KT / 16];
#pragma unroll
        for (int n = 0; n < KT / 16; n++) {
            sc[n] = omh_v4f{0.f, 0.f, 0.f, 0.f};
            const float *kp = Ks + (16 * n + l16) * LD + 4 * gq;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const omh_v4f kf = *reinterpret_cast<const omh_v4f *>(kp + 16 * c);
#pragma unroll
                for (int s = 0; s < 4; s++) sc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[s], q[c][s], sc[n], 0, 0, 0);
            }
        }
        // scores * hd^-1/2, causal mask, online softmax (qwen.c:410-414)
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < KT / 16; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kt + 16 * n + 4 * gq + i;
                sc[n][i] = key <= kmax ? sc[n][i] * a.scale : -INFINITY;
                mx = fmaxf(mx, sc[n][i]);
            }
        mx = omh_swap32_max(omh_swap16_max(mx));
        const float mn = fmaxf(m, mx);             // finite: key 0 is in every token's first tile
        const float corr = expf(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int n = 0; n < KT / 16; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[n][i] = expf(sc[n][i] - mn);
                ps += sc[n][i];
            }
        ps = omh_swap32_sum(omh_swap16_sum(ps));
        l = fmaf(l, corr, ps);
        m = mn;
        // O^T = corr O^T + V^T P^T (qwen.c:415-419)
#pragma unroll
        for (int j = 0; j < NC; j++) {
            o[j] = o[j] * corr;
#pragma unroll
            for (int n = 0; n < KT / 16; n++) {
                const float *vp = Vs + (16 * n + 4 * gq) * LD + 16 * j + l16;
#pragma unroll
                for (int s = 0; s < 4; s++) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vp[s * LD], sc[n][s], o[j], 0, 0, 0);
            }
        }
        if (kt + KT < nkeys) put(st ^ 1);
        __syncthreads();
    }
    // normalise and gate (qwen.c:420-421)
    if (!own || tq >= a.T) return;
    const float il = 1.f / l;
    const float *gate = a.qkv + (size_t)tq * a.ld_qkv + (size_t)h * 2 * HD + HD + 4 * gq;
    float *dst = a.ctx + ((size_t)tq * H + h) * HD + 4 * gq;
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const float4 gv = *reinterpret_cast<const float4 *>(gate + 16 * j);
        float4 r;
        r.x = o[j][0] * il * omh_sigmoid(gv.x);
        r.y = o[j][1] * il * omh_sigmoid(gv.y);
        r.z = o[j][2] * il * omh_sigmoid(gv.z);
        r.w = o[j][3] * il * omh_sigmoid(gv.w);
        *reinterpret_cast<float4 *>(dst + 16 * j) = r;
    }
}

// The same flash attention with every product as three bf16 products on
// the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation): each
// fp32 operand x splits as hi = bf16(x), lo = bf16(x - hi), so
// x = hi + lo to 2^-16 relative, and a.b = hi.hi + hi.lo + lo.hi with the
// dropped lo.lo term below 2^-16 |a||b|; per 32 keys a wave issues 96 such
// products against 256 fp32 ones.  K is staged into LDS as hi / lo planes
// row-major (32 head dims per 16-byte read), V transposed (V^T[dim][key],
// 8 keys per 16-byte read) with its keys in the order the probabilities
// already sit in the score product's registers: position 8 g + j of a
// V^T row holds key 16 (j / 4) + 4 g + j % 4, which lane group g of the
// B operand P^T holds as register j % 4 of its score sub-tile j / 4.  Rows
// are padded so that every 16-lane group's reads fall in distinct banks.
template <int HD>
struct Flash3Shape {
    static constexpr int KT = 32;                  // keys per tile
    // bytes of one bf16 K row.  The padding sets the LDS bank conflicts of the
    // 16-byte K reads (SQ_LDS_BANK_CONFLICT per T = 4096 dispatch at HD = 256):
    // 270.5 M cycles unpadded, 67.6 M with 16 / 48 / 64 bytes, 33.8 M with 32
    // or 96 bytes; 96 gave the fastest kernel (499-505 against 521-527 us
    // under the counters, the fastest of seven calls 539 against 554 us);
    // the two stages then take 156 KiB of LDS.
    static constexpr int KLD = 2 * HD + 96;
    static constexpr int VLD = 2 * KT + 16;        // bytes of one bf16 V^T row
    static constexpr int KPL = KT * KLD, VPL = HD * VLD;
    static constexpr int STAGE = 2 * KPL + 2 * VPL;   // K hi, K lo, V^T hi, V^T lo
    static constexpr size_t LDS = 2 * (size_t)STAGE;
    static constexpr int NS = HD / 32;             // 32-dim steps of q.k
    static constexpr int NJ = HD / 16;             // 16-dim output tiles
    static constexpr int PK = KT * HD / 4 / (8 * OMH_WAVE);         // K float4 pieces per thread
    static constexpr int PV = KT / 2 * HD / 4 / (8 * OMH_WAVE);     // V (key pair, 4 dims) units per thread
    static_assert(LDS <= 160 * 1024 && KLD % 16 == 0 && VLD % 16 == 0, "two stages in a CU's LDS, 16-byte rows");
};
typedef __bf16 omh_v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) | (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16;
}
__device__ __forceinline__ float bf16_rest(float x) { return x - (float)(__bf16)x; }

// One 32-key tile of K and V on its way to the flash kernel's LDS image: the
// fp32 rows of keys kt .. kt + 31 (past nkeys, the tile's first row again)
// into registers (load), then as bf16 hi / lo planes, K by rows and V
// transposed, in the Flash3Shape stage layout (put: to an LDS stage, or to
// a tile image in memory that the kernel later copies into LDS whole).
template <int HD>
struct Flash3Tile {
    using F = Flash3Shape<HD>;
    static constexpr int KT = F::KT, KLD = F::KLD, VLD = F::VLD, NT = 8 * OMH_WAVE;
    omh_v4f kr[F::PK], vr[F::PV][2];
    // V unit e: the key pair at V^T positions 2 pp, 2 pp + 1 (pp = e % 16) for
    // head dims 4 c .. 4 c + 3 (c = e / 16), so the 16 lanes of a position
    // pair sweep write one 64-byte run of a V^T row: no bank conflicts.
    // Position 8 g + j holds key 16 (j / 4) + 4 g + j % 4.
    static __device__ __forceinline__ int vkey(int pp) {
        const int pos = 2 * pp, g8 = pos / 8, j = pos % 8;
        return 16 * (j / 4) + 4 * g8 + j % 4;
    }
    __device__ __forceinline__ void load(const float *Kg, const float *Vg, int kt, int nkeys, int tid) {
        auto key_of = [&](int kk) { return (size_t)(kt + kk < nkeys ? kt + kk : kt); };
#pragma unroll
        for (int i = 0; i < F::PK; i++) {
            const int e = tid + NT * i, kk = e / (HD / 4), c = e % (HD / 4);
            kr[i] = *reinterpret_cast<const omh_v4f *>(Kg + key_of(kk) * HD + 4 * c);
        }
#pragma unroll
        for (int i = 0; i < F::PV; i++) {
            const int e = tid + NT * i, k0 = vkey(e % 16), c = e / 16;
            vr[i][0] = *reinterpret_cast<const omh_v4f *>(Vg + key_of(k0) * HD + 4 * c);
            vr[i][1] = *reinterpret_cast<const omh_v4f *>(Vg + key_of(k0 + 1) * HD + 4 * c);
        }
    }
    __device__ __forceinline__ void put(unsigned char *st, int tid) const {
        unsigned char *Kh = st, *Kl = st + F::KPL, *Vh = st + 2 * F::KPL, *Vl = Vh + F::VPL;
#pragma unroll
        for (int i = 0; i < F::PK; i++) {
            const int e = tid + NT * i, kk = e / (HD / 4), c = e % (HD / 4);
            const omh_v4f x = kr[i];
            uint2 hi, lo;
            hi.x = bf16_pair(x[0], x[1]);
            hi.y = bf16_pair(x[2], x[3]);
            lo.x = bf16_pair(bf16_rest(x[0]), bf16_rest(x[1]));
            lo.y = bf16_pair(bf16_rest(x[2]), bf16_rest(x[3]));
            *reinterpret_cast<uint2 *>(Kh + kk * KLD + 8 * c) = hi;
            *reinterpret_cast<uint2 *>(Kl + kk * KLD + 8 * c) = lo;
        }
#pragma unroll
        for (int i = 0; i < F::PV; i++) {
            const int e = tid + NT * i, pos = 2 * (e % 16), c = e / 16;
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const float x0 = vr[i][0][d], x1 = vr[i][1][d];
                *reinterpret_cast<uint32_t *>(Vh + (4 * c + d) * VLD + 2 * pos) = bf16_pair(x0, x1);
                *reinterpret_cast<uint32_t *>(Vl + (4 * c + d) * VLD + 2 * pos) = bf16_pair(bf16_rest(x0), bf16_rest(x1));
            }
        }
    }
};

// The tile images of keys 0 .. pos + T - 1 of the step's sequence, one
// workgroup per (kv head, tile): image (g, i) at a.img + (g * a.img_tiles +
// i) * STAGE holds exactly what attn_flash3_kernel stages in LDS for tile i.
template <int HD>
__global__ __launch_bounds__(8 * OMH_WAVE) void attn_tile_image_kernel(const AttnArgs a) {
    using F = Flash3Shape<HD>;
    const int g = blockIdx.x % a.KV, ti = blockIdx.x / a.KV;
    const size_t cache0 = ((size_t)a.seq * a.KV + g) * a.max_t;
    Flash3Tile<HD> t;
    t.load(a.Kc + cache0 * HD, a.Vc + cache0 * HD, ti * F::KT, a.pos + a.T, threadIdx.x);
    t.put(a.img + ((size_t)g * a.img_tiles + ti) * F::STAGE, threadIdx.x);
}

// IMG: each tile goes from its image (attn_tile_image_kernel) into LDS as
// whole 1 KiB runs (buffer loads to LDS), with no conversion in the kernel.
template <int HD, bool IMG>
__global__ __launch_bounds__(8 * OMH_WAVE) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_flash3_kernel(const AttnArgs a) {
    using F = Flash3Shape<HD>;
    constexpr int KT = F::KT, KLD = F::KLD, VLD = F::VLD, NS = F::NS, NJ = F::NJ;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem3[];
    const int H = a.H, KV = a.KV, grp = H / KV;
    const int nunit = (a.T + 15) / 16 * grp, wpg = (nunit + 7) / 8;
    const int g = blockIdx.x % KV, wi = wpg - 1 - (int)blockIdx.x / KV;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, gq = lane / 16;
    const bool own = 8 * wi + w < nunit;
    const int u = min(8 * wi + w, nunit - 1);
    const int tb = u / grp, h = g * grp + u % grp;
    const int tq = 16 * tb + l16;                  // this lane's query token (may be past T: not written)
    const int tlast = min(16 * (min(8 * wi + 7, nunit - 1) / grp) + 15, a.T - 1);
    const int nkeys = a.pos + tlast + 1;
    const int kmax = a.pos + tq;

    // q as the B operand of S^T: dims 32 s + 8 gq .. +7 of token tq, hi and lo
    omh_v8bf qh[NS], ql[NS];
    {
        const float *qr = a.qb + ((size_t)min(tq, a.T - 1) * H + h) * HD + 8 * gq;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float4 x0 = *reinterpret_cast<const float4 *>(qr + 32 * s);
            const float4 x1 = *reinterpret_cast<const float4 *>(qr + 32 * s + 4);
            const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                qh[s][j] = (__bf16)v[j];
                ql[s][j] = (__bf16)bf16_rest(v[j]);
            }
        }
    }
    const size_t cache0 = ((size_t)a.seq * KV + g) * a.max_t;
    const float *Kg = a.Kc + cache0 * HD, *Vg = a.Vc + cache0 * HD;
    Flash3Tile<HD> tile;
    // IMG: kv head g's tile images, F::STAGE bytes (whole 1 KiB runs) each
    static_assert(F::STAGE % 1024 == 0, "an image tile is whole 1 KiB runs");
    constexpr int NCH = F::STAGE / 1024;
    const __amdgpu_buffer_rsrc_t irs =
        omh_rsrc(IMG ? a.img + (size_t)g * a.img_tiles * F::STAGE : a.img, IMG ? a.img_tiles * F::STAGE : 0);
    auto copy = [&](int kt, int stage) __attribute__((always_inline)) {
        unsigned char *dst = smem3 + stage * F::STAGE;
        const int src = kt / KT * F::STAGE;
#pragma unroll
        for (int i = 0; i < (NCH + 7) / 8; i++) {
            const int c = w + 8 * i;
            if (c < NCH)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(irs, (__attribute__((address_space(3))) void *)(dst + c * 1024),
                                                         16, 16 * lane, src + c * 1024, 0, 0);
        }
    };
    auto load = [&](int kt) __attribute__((always_inline)) { tile.load(Kg, Vg, kt, nkeys, tid); };
    auto put = [&](int stage) __attribute__((always_inline)) { tile.put(smem3 + stage * F::STAGE, tid); };

    omh_v4f o[NJ];                                 // O^T: o[j][i] = O[token tq][dim 16 j + 4 gq + i]
#pragma unroll
    for (int j = 0; j < NJ; j++) o[j] = omh_v4f{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    if constexpr (IMG) {
        copy(0, 0);
        __builtin_amdgcn_s_waitcnt(0x0f70);     // vmcnt(0): this wave's copies have landed
    } else {
        load(0);
        put(0);
    }
    __syncthreads();
    for (int kt = 0, st = 0; kt < nkeys; kt += KT, st ^= 1) {
        // (stage st ^ 1 was last read before the barrier that ended the previous step)
        if (kt + KT < nkeys) {
            if constexpr (IMG) copy(kt + KT, st ^ 1);
            else load(kt + KT);
        }
        const unsigned char *sb = smem3 + st * F::STAGE;
        const unsigned char *Kh = sb, *Kl = sb + F::KPL, *Vh = sb + 2 * F::KPL, *Vl = Vh + F::VPL;
        // S^T for keys kt + 16 n + 4 gq + i (register i of sc[n]), query row tq
        omh_v4f sc[KT / 16];
#pragma unroll
        for (int n = 0; n < KT / 16; n++) {
            sc[n] = omh_v4f{0.f, 0.f, 0.f, 0.f};
            const size_t ro = (size_t)(16 * n + l16) * KLD + 16 * gq;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const omh_v8bf kh = *reinterpret_cast<const omh_v8bf *>(Kh + ro + 64 * s);
                const omh_v8bf kl = *reinterpret_cast<const omh_v8bf *>(Kl + ro + 64 * s);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[s], sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[s], sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[s], sc[n], 0, 0, 0);
            }
        }
        // scores * hd^-1/2, causal mask, online softmax (qwen.c:410-414)
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < KT / 16; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kt + 16 * n + 4 * gq + i;
                sc[n][i] = key <= kmax ? sc[n][i] * a.scale : -INFINITY;
                mx = fmaxf(mx, sc[n][i]);
            }
        mx = omh_swap32_max(omh_swap16_max(mx));
        const float mn = fmaxf(m, mx);             // finite: key 0 is in every token's first tile
        // e^(s - mn) as 2^((s - mn) log2 e) on the hardware exp2 (a masked
        // score, -inf, gives 0; the first tile's corr, 2^-inf, 0)
        const float corr = __builtin_amdgcn_exp2f((m - mn) * 1.4426950408889634f);
        float ps = 0.f;
        omh_v8bf ph, pl;                           // P^T as the B operand: j = 4 n + i
#pragma unroll
        for (int n = 0; n < KT / 16; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = __builtin_amdgcn_exp2f((sc[n][i] - mn) * 1.4426950408889634f);
                ps += pv;
                ph[4 * n + i] = (__bf16)pv;
                pl[4 * n + i] = (__bf16)bf16_rest(pv);
            }
        ps = omh_swap32_sum(omh_swap16_sum(ps));
        l = fmaf(l, corr, ps);
        m = mn;
        // O^T = corr O^T + V^T P^T (qwen.c:415-419); the rescale only when a
        // row's max moved (corr = 1 otherwise)
        if (__builtin_amdgcn_ballot_w64(corr != 1.f))
#pragma unroll
            for (int j = 0; j < NJ; j++) o[j] = o[j] * corr;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const size_t ro = (size_t)(16 * j + l16) * VLD + 16 * gq;
            const omh_v8bf vh = *reinterpret_cast<const omh_v8bf *>(Vh + ro);
            const omh_v8bf vl = *reinterpret_cast<const omh_v8bf *>(Vl + ro);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph, o[j], 0, 0, 0);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl, o[j], 0, 0, 0);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph, o[j], 0, 0, 0);
        }
        if constexpr (IMG) __builtin_amdgcn_s_waitcnt(0x0f70);
        else if (kt + KT < nkeys) put(st ^ 1);
        __syncthreads();
    }
    // normalise and gate (qwen.c:420-421)
    if (!own || tq >= a.T) return;
    const float il = 1.f / l;
    const float *gate = a.qkv + (size_t)tq * a.ld_qkv + (size_t)h * 2 * HD + HD + 4 * gq;
    float *dst = a.ctx + ((size_t)tq * H + h) * HD + 4 * gq;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float4 gv = *reinterpret_cast<const float4 *>(gate + 16 * j);
        float4 r;
        r.x = o[j][0] * il * omh_sigmoid(gv.x);
        r.y = o[j][1] * il * omh_sigmoid(gv.y);
        r.z = o[j][2] * il * omh_sigmoid(gv.z);
        r.w = o[j][3] * il * omh_sigmoid(gv.w);
        *reinterpret_cast<float4 *>(dst + 16 * j) = r;
    }
}

// One workgroup per (token, head, 64 columns): the CW waves take every
// CW-th split, lane = column, then sum through LDS.
constexpr int kCombineWaves = 8;
template <int HD>
__global__ __launch_bounds__(kCombineWaves * OMH_WAVE) void attn_combine_kernel(const AttnArgs a) {
    constexpr int NCB = HD < OMH_WAVE ? 1 : HD / OMH_WAVE;     // column blocks per head
    constexpr int CW = kCombineWaves;
    __shared__ float so[CW][OMH_WAVE], sl[CW];
    const int th = blockIdx.x / NCB, cb = blockIdx.x % NCB;
    const int t = th / a.H, h = th % a.H, ns = a.ns;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int j = cb * OMH_WAVE + lane;
    const size_t pb = (size_t)th * ns;
    float M = -INFINITY;
    for (int s = lane; s < ns; s += OMH_WAVE) M = fmaxf(M, a.pml[2 * (pb + s)]);
    M = wave_max(M);
    float L = 0.f, o = 0.f;
    const int jc = j < HD ? j : HD - 1;
#pragma unroll 8
    for (int s = wave; s < ns; s += CW) {          // an empty split: m = -inf, weight 0, zero partial
        const float wgt = expf(a.pml[2 * (pb + s)] - M);
        L = fmaf(a.pml[2 * (pb + s) + 1], wgt, L);
        o = fmaf(a.po[(pb + s) * HD + jc], wgt, o);
    }
    so[wave][lane] = o;
    if (lane == 0) sl[wave] = L;
    __syncthreads();
    if (wave == 0 && j < HD) {
        float ls = 0.f, os = 0.f;                  // split 0 always holds key 0: ls > 0
#pragma unroll
        for (int w = 0; w < CW; w++) {
            ls += sl[w];
            os += so[w][lane];
        }
        const float g = a.qkv[(size_t)t * a.ld_qkv + (size_t)h * 2 * HD + HD + j];
        a.ctx[((size_t)t * a.H + h) * HD + j] = os / ls * omh_sigmoid(g);
    }
}

template <int HD>
hipError_t launch_attn_d(const AttnArgs &a, hipStream_t st) {
    static const bool lds_ok = [] {
        bool ok = true;
        if constexpr (HD >= 64) {
            for (const void *f : {(const void *)attn_split_mfma_kernel<HD, false>, (const void *)attn_split_mfma_kernel<HD, true>})
                ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)MfmaSplitShape<HD>::LDS) == hipSuccess;
        } else {
            for (const void *f : {(const void *)attn_split_kernel<HD, 1>, (const void *)attn_split_kernel<HD, 2>,
                                  (const void *)attn_split_kernel<HD, 3>, (const void *)attn_split_kernel<HD, 4>,
                                  (const void *)attn_split_kernel<HD, 1, true>, (const void *)attn_split_kernel<HD, 2, true>,
                                  (const void *)attn_split_kernel<HD, 3, true>, (const void *)attn_split_kernel<HD, 4, true>})
                ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)AttnShape<HD>::LDS) == hipSuccess;
        }
        return ok;
    }();
    if (!lds_ok) return hipErrorInvalidValue;
    static_assert(kAttnMaxGroup <= 4 * AttnShape<HD>::NW, "heads per wave");
    // decode steps: the prep is done inside the split kernel (OMH_ATTN_FUSE=0: its own launch, for comparison)
    const bool flash = HD >= 128 && attn_uses_flash(a.T, HD);
    const bool fuse = a.T == 1 && !flash && fuse_prep();
    if (!fuse) hipLaunchKernelGGL((attn_prep_kernel<HD>), dim3((unsigned)a.T), dim3(kPrepWaves * OMH_WAVE), 0, st, a);
    if constexpr (HD >= 128) {
        if (attn_uses_flash(a.T, HD)) {
            const int wpg = ((a.T + 15) / 16 * (a.H / a.KV) + 7) / 8;
            const dim3 grid((unsigned)(a.KV * wpg)), blk(8 * OMH_WAVE);
            if (flash_fp32()) {
                static const bool ok = hipFuncSetAttribute((const void *)attn_flash_kernel<HD>,
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)FlashShape<HD>::LDS) == hipSuccess;
                if (!ok) return hipErrorInvalidValue;
                hipLaunchKernelGGL((attn_flash_kernel<HD>), grid, blk, FlashShape<HD>::LDS, st, a);
            } else {
                static const bool ok =
                    hipFuncSetAttribute((const void *)attn_flash3_kernel<HD, false>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)Flash3Shape<HD>::LDS) == hipSuccess &&
                    hipFuncSetAttribute((const void *)attn_flash3_kernel<HD, true>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)Flash3Shape<HD>::LDS) == hipSuccess;
                if (!ok) return hipErrorInvalidValue;
                if (a.img) {
                    // the images of every tile of keys 0 .. pos + T - 1, then the kernel copying them
                    const long tiles = ((long)a.pos + a.T + Flash3Shape<HD>::KT - 1) / Flash3Shape<HD>::KT;
                    if (a.img_tiles != tiles || (size_t)tiles * Flash3Shape<HD>::STAGE > (size_t)INT32_MAX)
                        return hipErrorInvalidValue;
                    hipLaunchKernelGGL((attn_tile_image_kernel<HD>), dim3((unsigned)(a.KV * tiles)), blk, 0, st, a);
                    hipLaunchKernelGGL((attn_flash3_kernel<HD, true>), grid, blk, Flash3Shape<HD>::LDS, st, a);
                } else {
                    hipLaunchKernelGGL((attn_flash3_kernel<HD, false>), grid, blk, Flash3Shape<HD>::LDS, st, a);
                }
            }
            return hipGetLastError();
        }
    }
    if constexpr (HD >= 64) {
        // the K / V slices of a (sequence, kv head) are addressed by 32-bit byte offsets
        if ((size_t)a.max_t * HD * sizeof(float) > (size_t)INT32_MAX) return hipErrorInvalidValue;
        const dim3 grid((unsigned)(a.ns * a.KV * a.T)), blk(MfmaSplitShape<HD>::NW * OMH_WAVE);
        const size_t lds = MfmaSplitShape<HD>::LDS;
        if (fuse) hipLaunchKernelGGL((attn_split_mfma_kernel<HD, true>), grid, blk, lds, st, a);
        else hipLaunchKernelGGL((attn_split_mfma_kernel<HD, false>), grid, blk, lds, st, a);
    } else {
        const dim3 grid((unsigned)(a.ns * a.KV * a.T)), blk(AttnShape<HD>::NW * OMH_WAVE);
        const size_t lds = AttnShape<HD>::LDS;
        const int gpw = (a.H / a.KV + AttnShape<HD>::NW - 1) / AttnShape<HD>::NW;
        if (fuse) {
            switch (gpw) {
            case 1: hipLaunchKernelGGL((attn_split_kernel<HD, 1, true>), grid, blk, lds, st, a); break;
            case 2: hipLaunchKernelGGL((attn_split_kernel<HD, 2, true>), grid, blk, lds, st, a); break;
            case 3: hipLaunchKernelGGL((attn_split_kernel<HD, 3, true>), grid, blk, lds, st, a); break;
            default: hipLaunchKernelGGL((attn_split_kernel<HD, 4, true>), grid, blk, lds, st, a); break;
            }
        } else {
            switch (gpw) {
            case 1: hipLaunchKernelGGL((attn_split_kernel<HD, 1>), grid, blk, lds, st, a); break;
            case 2: hipLaunchKernelGGL((attn_split_kernel<HD, 2>), grid, blk, lds, st, a); break;
            case 3: hipLaunchKernelGGL((attn_split_kernel<HD, 3>), grid, blk, lds, st, a); break;
            default: hipLaunchKernelGGL((attn_split_kernel<HD, 4>), grid, blk, lds, st, a); break;
            }
        }
    }
    constexpr int NCB = HD < OMH_WAVE ? 1 : HD / OMH_WAVE;
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3((unsigned)(a.T * a.H * NCB)), dim3(kCombineWaves * OMH_WAVE), 0, st, a);
    return hipGetLastError();
}

}  // namespace

bool attn_uses_flash(int T, int hd) {
    if (const char *e = getenv("OMH_ATTN_FLASH"))
        if (e[0] == '0') return false;
    return T >= kFlashMinT && (hd == 128 || hd == 256);
}

template <int HD>
size_t flash_image_bytes_d(int KV, int pos, int T, int *tiles) {
    using F = Flash3Shape<HD>;
    const size_t n = ((size_t)pos + T + F::KT - 1) / F::KT;
    // one kv head's images are addressed with 32-bit buffer offsets: longer
    // steps stage their tiles in the kernel
    if (n * F::STAGE > (size_t)INT32_MAX) return 0;
    *tiles = (int)n;
    return (size_t)KV * n * F::STAGE;
}

size_t attn_flash_image_bytes(int hd, int KV, int pos, int T, int *tiles) {
    *tiles = 0;
    if (!attn_uses_flash(T, hd) || T < kFlashImageMinT || flash_fp32() || flash_reg()) return 0;
    return hd == 256 ? flash_image_bytes_d<256>(KV, pos, T, tiles) : flash_image_bytes_d<128>(KV, pos, T, tiles);
}

bool attn_supported(int hd, int H, int KV, int rot) {
    return (hd == 32 || hd == 64 || hd == 128 || hd == 256) && KV >= 1 && H >= KV && H % KV == 0 &&
           H / KV <= kAttnMaxGroup && rot >= 0 && rot <= hd && rot % 2 == 0;
}

void attn_plan(int pos, int T, int KV, int &ns, int &kps) {
    const long nmax = (long)pos + T;                       // keys the last token sees
    const long per = (long)KV * T;
    const long want = per >= 256 ? 1 : (256 + per - 1) / per;   // splits for >= 256 workgroups (one per CU)
    long k = (nmax + want - 1) / want;
    k = (k + 63) / 64 * 64;
    kps = (int)k;
    ns = (int)((nmax + k - 1) / k);
}

hipError_t launch_attn(const AttnArgs &a, int hd, hipStream_t st) {
    if (a.T <= 0) return hipSuccess;
    if (!attn_supported(hd, a.H, a.KV, a.rot) || a.ns < 1 || a.kps < 1 || (long)a.ns * a.kps < (long)a.pos + a.T ||
        a.pos < 0 || (long)a.pos + a.T > a.max_t)
        return hipErrorInvalidValue;
    switch (hd) {
    case 32: return launch_attn_d<32>(a, st);
    case 64: return launch_attn_d<64>(a, st);
    case 128: return launch_attn_d<128>(a, st);
    default: return launch_attn_d<256>(a, st);
    }
}

}  // namespace omh
