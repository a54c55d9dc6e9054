// gdn_decode.hip — one-token GDN core for many (layer, sequence) slots.
//
// Fuses, for one token, the decode-side stages of the layer core
// (overhang engines/qwen.c:307-358):
//   (1) causal conv1d update (kernel K) + SiLU, per-head q/k L2 norm and q
//       scale, gates g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
//   (3) the gated delta-rule update of the fp32 state S[kd][vd] of each
//       value head:  S <- gamma S;  kv = S^T k;  delta = beta (v - kv);
//       S <- S + k delta^T;  o = S^T q;
//   (4) the gated RMSNorm  o * rsqrt(mean(o^2) + eps) * gnorm * silu(z).
//
// The step is bound by HBM: each value head's state is read once and
// written once (2*kd*vd*4 bytes), with streaming (nontemporal) accesses.
// One pass over the state computes both column sums S^T k and S^T q of
// the old state; with them
//     kv = gamma S^T k,   delta = beta (v - kv),
//     o  = gamma S^T q + (k.q) delta        (= (gamma S + k delta^T)^T q),
// so a head needs a single cross-row reduction, and the second pass only
// forms gamma S + k delta^T and streams it back.  q and k are kept as raw
// conv outputs; their L2-norm factors (qwen.c:153-157, 326-329) are applied
// to the sums and to delta instead of to every element.
//
// Two kernels share that contract:
//  * paired (large launches): one workgroup per (layer, sequence, key head)
//    handles the rep = vh/kh value heads that share the key head.  The
//    q/k conv + norm is done once for all of them, and the state of the
//    next value head is loaded while the current one is reduced and stored,
//    so every workgroup keeps reads in flight under its own writes.
//  * sliced (small launches): one workgroup per value head, or per column
//    slice of one.  The delta rule couples only the rows of one column, so
//    a head may split into NCS slices.  The gated RMSNorm needs the whole
//    row of o: either each slice writes o * gnorm * silu(z) and its partial
//    sum of squares of o, and the consumer applies 1 / rms (a whole-layer
//    step at up to 4 tokens: out_proj's GEMV, as it loads x), or each slice
//    publishes its raw o and partial sum (device-coherent atomic stores)
//    and the last slice of the head to arrive (arrival counter) applies the
//    norm to all vd columns.  Both sum the partials in slice order, so the
//    result does not depend on arrival order.
//
// Conv history lives in a per-channel ring (omh_internal.h): readers use
// the K-1 history slots (the sliced kernel requests every slot and picks by
// the phase once it arrives), the single owner of a channel writes the new
// input into the free slot.
//
// When the step feeds an int8 out_proj of more than 4 tokens, the epilogue
// also writes the gated output as that projection's x planes (int8 x 3 with
// a scale per 128-wide block, or exact bf16 x 3 with 64-wide block sums;
// write_x), so the projection needs no split launch.  A launch covers
// sequences b0 .. b0+B-1; the host runs one layer's large batch as several
// launches that each fit one round of resident workgroups.
//
// Thread layout: TPB threads hold RPT rows x 4 adjacent columns (a float4)
// of a head (or slice); a wavefront's loads cover whole consecutive row
// segments.  Column sums over rows are butterflies across the row groups of
// a wave (DPP row operations and permlane swaps, omh_lane_sum_from), then
// across waves through LDS.
#include "omh_device.h"
#include "omh_internal.h"

namespace omh {
namespace {

constexpr int kMaxRep = 8;            // value heads per key head, paired kernel

// MAXT: the most threads per workgroup.  256 for the paired kernel, whose
// launches put two workgroups on every CU; 512 for the sliced kernel, whose
// small launches leave most CUs idle, so a head's tile is worth more waves
// (one layer at B = 1 on MI355X: 5.9 us with 512 threads per value head,
// 7.6 us with 256, 7.8 us with 1024).
template <int KD, int CW, int MAXT = 256>
struct TileShape {
    static constexpr int C4 = CW / 4;                       // float4 columns per row
    static constexpr int TPB_RAW = KD * C4 / 4;             // aim for 4 float4 per thread
    static constexpr int TPB = TPB_RAW < 64 ? 64 : (TPB_RAW > MAXT ? MAXT : TPB_RAW);
    static constexpr int RG = TPB / C4;                     // row groups
    static constexpr int RPT = KD / RG;                     // rows per thread
    static constexpr int NW = TPB / OMH_WAVE;
    static_assert(CW % 4 == 0 && C4 >= 1 && C4 <= OMH_WAVE, "tile layout");
    static_assert((C4 & (C4 - 1)) == 0 && TPB % C4 == 0, "tile layout");
    static_assert(RG >= 1 && KD % RG == 0 && RPT >= 1, "row layout");
};

constexpr int kSliceMaxT = 512;       // the sliced kernel's MAXT

// Whether TileShape<KD, VD / NCS, kSliceMaxT> with the sliced norm epilogue is valid.
constexpr bool slice_valid(int KD, int VD, int NCS) {
    if (NCS < 1 || VD % NCS != 0 || (VD / NCS) % 4 != 0 || NCS > kMaxSlices) return false;
    const int c4 = VD / NCS / 4;
    if (c4 < 1 || c4 > OMH_WAVE || (c4 & (c4 - 1)) != 0) return false;
    const int raw = KD * c4 / 4;
    const int tpb = raw < 64 ? 64 : (raw > kSliceMaxT ? kSliceMaxT : raw);
    const int rg = tpb / c4;
    return tpb % c4 == 0 && rg <= KD && KD % rg == 0 && VD / 4 <= tpb;
}

template <int C4>
__device__ __forceinline__ float4 f4_lane_sum_from(float4 x) {
    x.x = omh_lane_sum_from<C4>(x.x);
    x.y = omh_lane_sum_from<C4>(x.y);
    x.z = omh_lane_sum_from<C4>(x.z);
    x.w = omh_lane_sum_from<C4>(x.w);
    return x;
}
__device__ __forceinline__ float4 f4_add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Sum two float4 over the row groups of the workgroup (red: [NW][2][C4]).
template <int C4, int NW>
__device__ __forceinline__ void colsum2(float4 &a, float4 &b, float4 (*red)[2][C4], int wave, int lane, int c4) {
    a = f4_lane_sum_from<C4>(a);
    b = f4_lane_sum_from<C4>(b);
    if constexpr (NW > 1) {
        if (lane < C4) { red[wave][0][c4] = a; red[wave][1][c4] = b; }
        omh_lds_barrier();
        a = red[0][0][c4];
        b = red[0][1][c4];
#pragma unroll
        for (int w = 1; w < NW; w++) { a = f4_add(a, red[w][0][c4]); b = f4_add(b, red[w][1][c4]); }
    }
}

// FAST: the exp2 / reciprocal SiLU (omh_silu_fast) instead of the
// correctly rounded one (see qk_factors)
template <bool FAST>
__device__ __forceinline__ float silu_of(float z) { return FAST ? omh_silu_fast(z) : omh_silu(z); }
template <bool FAST>
__device__ __forceinline__ float4 gated(float4 o, float rn, float4 gn, float4 zz) {
    float4 y;
    y.x = o.x * rn * gn.x * silu_of<FAST>(zz.x);
    y.y = o.y * rn * gn.y * silu_of<FAST>(zz.y);
    y.z = o.z * rn * gn.z * silu_of<FAST>(zz.z);
    y.w = o.w * rn * gn.w * silu_of<FAST>(zz.w);
    return y;
}

// Conv inputs of the NIT channels a thread handles, loaded into registers
// in one batch (vector memory operations complete in issue order for the
// wait counter, so the first use waits for exactly these and what came
// before them).  History is right-aligned: h[it][m] is the input
// kConvRing-1-m tokens back, in ring slot (ph + 1 + m) mod kConvRing; the
// taps are stored right-aligned the same way, so tap m multiplies h[m] and
// the last tap the new input.  ALL: every ring slot is requested without
// the phase (one slot more per channel), and pick() takes the history slots
// out of them once the phase has arrived, so no load waits for the phase.
template <int NIT, bool ALL = false>
struct ConvIn {
    static constexpr int NH = kConvRing - 1;
    float x[NIT], h[NIT][NH];
    float r[ALL ? NIT : 1][kConvRing];
    float4 w[NIT];
    int gch[NIT];

    // gch_of(c) maps the workgroup's channel c < nch to a global channel.
    // The loads are branch-free (out-of-range slots load channel 0 and are
    // marked gch = -1; without ALL, history slots a K < kConvRing kernel
    // does not use repeat the first used slot's address), so the compiler's
    // wait counts stay exact and no unused bytes are fetched.
    template <typename F>
    __device__ __forceinline__ void load(F gch_of, int nch, int tid, int tpb, const float *qkv, const float *conv_w,
                                         const float *ring, int conv_dim, int seq, int ph, int K) {
        const int m0 = kConvRing - K;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int c = tid + it * tpb;
            const int g = gch_of(c < nch ? c : 0);
            gch[it] = c < nch ? g : -1;
            x[it] = qkv[g];
            w[it] = *reinterpret_cast<const float4 *>(conv_w + (size_t)g * kConvRing);
            const float *rs = ring + ring_at(seq, 0, g, conv_dim);
            if constexpr (ALL) {
#pragma unroll
                for (int q = 0; q < kConvRing; q++) r[it][q] = rs[(size_t)q * conv_dim];
            } else {
#pragma unroll
                for (int m = 0; m < NH; m++)
                    h[it][m] = rs[(size_t)((ph + 1 + (m < m0 ? m0 : m)) & (kConvRing - 1)) * conv_dim];
            }
        }
    }
    // ALL: the history slots of phase ph (the same slots load() reads
    // without ALL), by selects on the wave-uniform slot index.
    __device__ __forceinline__ void pick(int ph, int K) {
        static_assert(ALL, "pick() needs every slot loaded");
        const int m0 = kConvRing - K;
#pragma unroll
        for (int m = 0; m < NH; m++) {
            const int q = (ph + 1 + (m < m0 ? m0 : m)) & (kConvRing - 1);
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                float v = r[it][0];
#pragma unroll
                for (int qq = 1; qq < kConvRing; qq++) v = q == qq ? r[it][qq] : v;
                h[it][m] = v;
            }
        }
    }
    // conv1d + SiLU (op order as engines/qwen.c:311-319) of the it-th channel.
    template <bool FAST>
    __device__ __forceinline__ float conv(int it, int K) const {
        const float wt[kConvRing] = {w[it].x, w[it].y, w[it].z, w[it].w};
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < NH; m++)
            if (m >= kConvRing - K) acc += wt[m] * h[it][m];
        acc += wt[kConvRing - 1] * x[it];
        return silu_of<FAST>(acc);
    }
    // Append the new input: it goes to the free slot of phase ph.
    __device__ __forceinline__ void append(int it, float *ring, int conv_dim, int seq, int ph) const {
        ring[ring_at(seq, ph & (kConvRing - 1), gch[it], conv_dim)] = x[it];
    }
};

// L2-norm factors of the raw conv outputs q~, k~ of a key head, computed by
// every wave from LDS: rq = (|q~|^2 + 1e-6)^-1/2 kd^-1/2 (the q scale),
// rk = (|k~|^2 + 1e-6)^-1/2, and kq = q^.k^ (qwen.c:153-157, 326-329).
// FAST (the sliced kernel): the hardware reciprocal square root here and in
// the gated norm, and the exp2 / reciprocal SiLU, each within a few ulp.  In
// a small launch a workgroup's step is a chain of dependent instructions on
// one wave per SIMD, and the correctly rounded forms are some 40
// instructions each: 35B engine chain at B = 1 on MI355X 16.66 -> 16.20 us
// per layer.  The paired kernel keeps the correctly rounded forms: its
// 30-layer launch ran 22.8 -> 23.4 us with the fast ones (its workgroups'
// state writes then start while others still read; mixing the two costs
// HBM turnarounds).
template <int KD, bool FAST>
__device__ __forceinline__ void qk_factors(const float *s_q, const float *s_k, int lane, float &rq, float &rk,
                                           float &kq) {
    float sq = 0.f, sk = 0.f, sqk = 0.f;
    for (int i = lane; i < KD; i += OMH_WAVE) {
        const float q = s_q[i], k = s_k[i];
        sq += q * q;
        sk += k * k;
        sqk += q * k;
    }
    sq = omh_lane_sum_below<OMH_WAVE>(sq);
    sk = omh_lane_sum_below<OMH_WAVE>(sk);
    sqk = omh_lane_sum_below<OMH_WAVE>(sqk);
    rq = (FAST ? rsqrtf(sq + 1e-6f) : 1.f / sqrtf(sq + 1e-6f)) * (1.f / sqrtf((float)KD));
    rk = FAST ? rsqrtf(sk + 1e-6f) : 1.f / sqrtf(sk + 1e-6f);
    kq = sqk * rq * rk;
}

// Phase bookkeeping of the ring, per sequence: launch reads phase[epoch],
// writes phase[1 - epoch]; sequences outside the launch (outside
// [b0, b0 + B)) carry theirs over.
__device__ __forceinline__ void advance_phase(const LayerPtrs &L, int b0, int B, int seq, bool writer, bool copier,
                                              int ph, int tid, int tpb) {
    if (writer && tid == 0) L.phase[(1 - L.epoch) * L.max_seqs + seq] = (ph + 1) & (kConvRing - 1);
    if (copier)
        for (int bb = tid; bb < L.max_seqs; bb += tpb)
            if (bb < b0 || bb >= b0 + B) L.phase[(1 - L.epoch) * L.max_seqs + bb] = L.phase[L.epoch * L.max_seqs + bb];
}

// Per-head scalars of the delta rule.
struct HeadCoef {
    float gam, beta;      // decay gamma = e^g and beta
    float rk, rq, kq;     // key head's norm factors (qk_factors)
};

// Pass 1: column sums of S k~ and S q~ over this thread's rows, reduced over
// the workgroup, give kv, delta and o.  Pass 2: S <- gamma S + k~ (rk delta)^T,
// streamed back.  Returns o (before the gated norm).
template <int KD, int VD, int RG, int RPT, int C4, int NW>
__device__ __forceinline__ float4 delta_rule(float4 (&s)[RPT], float *Sp, const float *s_q, const float *s_k,
                                             float4 vv, const HeadCoef &hc, float4 (*red)[2][C4], int wave,
                                             int lane, int c4, int rg) {
    float4 ak = f4_zero(), aq = f4_zero();
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        const int i = rg + RG * m;
        ak = f4_fma(s[m], s_k[i], ak);
        aq = f4_fma(s[m], s_q[i], aq);
    }
    colsum2<C4, NW>(ak, aq, red, wave, lane, c4);
    const float4 kv = f4_scale(ak, hc.gam * hc.rk);
    const float4 delta = f4_scale(f4_sub(vv, kv), hc.beta);
    const float4 o = f4_fma(delta, hc.kq, f4_scale(aq, hc.gam * hc.rq));
    const float4 d2 = f4_scale(delta, hc.rk);
    const __amdgpu_buffer_rsrc_t rs = omh_rsrc(Sp, KD * VD * 4);
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        const int i = rg + RG * m;
        s[m] = f4_fma(d2, s_k[i], f4_scale(s[m], hc.gam));
        omh_st_stream_buf(rs, (i * VD + c4 * 4) * 4, s[m]);
    }
    return o;
}

// ------------------------------------------------------------- paired kernel
template <int KD, int VD>
struct PairShape : TileShape<KD, VD> {};

template <int KD, int VD, int RPT>
__device__ __forceinline__ void load_head(float4 (&s)[RPT], const float *Sp, int rg, int c4) {
    using Sh = PairShape<KD, VD>;
    static_assert(RPT == Sh::RPT, "tile rows");
    const __amdgpu_buffer_rsrc_t rs = omh_rsrc(Sp, KD * VD * 4);
#pragma unroll
    for (int m = 0; m < RPT; m++) s[m] = omh_ld_stream_buf(rs, ((rg + Sh::RG * m) * VD + c4 * 4) * 4);
}

// Where the core output also goes, when the decode step feeds an int8
// out_proj: the projection scratch's bf16 planes and block sums (xpiece
// layout, T tokens of I = vh * vd inputs).  null xb: not written.
struct PlaneOut {
    uint16_t *xb;
    int T, I;
    bool i8;
};

// Columns col .. col+3 (= 4 * c4 of a head starting at a multiple of 64) of
// token tok's output y, split exactly into three bf16 terms (hi = bf16(y),
// mid = bf16(y - hi), lo = the rest), and the sums of its 64-wide column
// blocks: a block is 16 lanes with consecutive c4, all active here.
__device__ __forceinline__ void write_planes(const PlaneOut &po, int tok, int col, int c4, float4 y) {
    typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
    const float v[4] = {y.x, y.y, y.z, y.w};
    v4bf hi, mid, lo;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        hi[j] = (__bf16)v[j];
        const float r1 = v[j] - (float)hi[j];
        mid[j] = (__bf16)r1;
        lo[j] = (__bf16)(r1 - (float)mid[j]);
    }
    const size_t plane = (size_t)po.T * po.I, o = xpiece(col / 8, tok, po.T, po.I) + col % 8;
    *reinterpret_cast<v4bf *>(po.xb + o) = hi;
    *reinterpret_cast<v4bf *>(po.xb + plane + o) = mid;
    *reinterpret_cast<v4bf *>(po.xb + 2 * plane + o) = lo;
    float sm = (y.x + y.y) + (y.z + y.w);
    sm += __shfl_xor(sm, 1, OMH_WAVE);
    sm += __shfl_xor(sm, 2, OMH_WAVE);
    sm += __shfl_xor(sm, 4, OMH_WAVE);
    sm += __shfl_xor(sm, 8, OMH_WAVE);
    if (c4 % 16 == 0) reinterpret_cast<float *>(po.xb + 3 * plane)[(size_t)tok * (po.I / 64) + col / 64] = sm;
}

// The same columns as int8 planes with the scale of their 128-wide block
// (i8_off layout, omh_i8_split): a block is 32 lanes with consecutive c4,
// all active here (vd a multiple of 128).
__device__ __forceinline__ void write_planes_i8(const PlaneOut &po, int tok, int col, int c4, float4 y) {
    float m = fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, OMH_WAVE));
    const int E = omh_i8_exponent(m);
    char4 a, b, c;
    int8_t t1, t2, t3;
    omh_i8_split(y.x, E, t1, t2, t3); a.x = t1; b.x = t2; c.x = t3;
    omh_i8_split(y.y, E, t1, t2, t3); a.y = t1; b.y = t2; c.y = t3;
    omh_i8_split(y.z, E, t1, t2, t3); a.z = t1; b.z = t2; c.z = t3;
    omh_i8_split(y.w, E, t1, t2, t3); a.w = t1; b.w = t2; c.w = t3;
    int8_t *X = reinterpret_cast<int8_t *>(po.xb);
    const size_t plane = i8_plane_bytes(po.T, po.I), o = i8_off(col, tok, po.T);
    *reinterpret_cast<char4 *>(X + o) = a;
    *reinterpret_cast<char4 *>(X + plane + o) = b;
    *reinterpret_cast<char4 *>(X + 2 * plane + o) = c;
    if (c4 % 32 == 0) reinterpret_cast<float *>(X + kI8Planes * plane)[(size_t)(col / kI8Blk) * po.T + tok] = ldexpf(1.f, E);
}

__device__ __forceinline__ void write_x(const PlaneOut &po, int tok, int col, int c4, float4 y) {
    if (po.i8) write_planes_i8(po, tok, col, c4, y);
    else write_planes(po, tok, col, c4, y);
}

// Delta rule + gated norm of one value head of the workgroup.
template <int KD, int VD, int RPT, int C4>
__device__ __forceinline__ void paired_head(float4 (&s)[RPT], float *Sp, float *core, const float *s_q,
                                            const float *s_k, const float *s_v, const float *s_z,
                                            const HeadCoef &hc, float4 gn, float eps, float4 (*red)[2][C4],
                                            int wave, int lane, int c4, int rg, const PlaneOut &po, int tok,
                                            int col0) {
    using Sh = PairShape<KD, VD>;
    static_assert(RPT == Sh::RPT && C4 == Sh::C4, "tile shape");
    const float4 vv = *reinterpret_cast<const float4 *>(&s_v[c4 * 4]);
    const float4 o = delta_rule<KD, VD, Sh::RG, RPT, C4, Sh::NW>(s, Sp, s_q, s_k, vv, hc, red, wave, lane, c4, rg);
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = omh_lane_sum_below<C4>(ss);
    if (rg == 0) {
        const float rn = 1.f / sqrtf(ss / (float)VD + eps);     // qwen.c:353-357
        const float4 zz = *reinterpret_cast<const float4 *>(&s_z[c4 * 4]);
        const float4 y = gated<false>(o, rn, gn, zz);
        *reinterpret_cast<float4 *>(core + c4 * 4) = y;
        if constexpr (VD % 64 == 0)
            if (po.xb) write_x(po, tok, col0 + c4 * 4, c4, y);
    }
}

template <int KD, int VD, int REPMAX>
__global__ __launch_bounds__((PairShape<KD, VD>::TPB))
void gdn_decode_paired_kernel(const DecodeArgs args) {
    using Sh = PairShape<KD, VD>;
    constexpr int TPB = Sh::TPB, C4 = Sh::C4, NW = Sh::NW;
    constexpr int NIT = (2 * KD + REPMAX * VD + TPB - 1) / TPB;   // conv channels per thread
    constexpr int NZ = (REPMAX * VD + TPB - 1) / TPB;             // z values per thread

    const int hk = blockIdx.x;                   // key head
    const int b = blockIdx.y;                    // token row of the launch
    const int seq = args.b0 + b;                 // sequence (state slot)
    const int l = blockIdx.z;                    // layer slot
    const LayerPtrs &L = args.L[l];
    // rep comes precomputed with the head counts: the state address then
    // needs no arithmetic on loaded values beyond a multiply, so the layer's
    // state pointer and the counts are requested together and the first
    // state request waits for one argument round trip.
    float *const Sl = L.S;
    const int kh = args.kh, vh = args.vh, K = args.K, rep = args.rep;
    __builtin_amdgcn_sched_barrier(0);
    const int h0 = hk * rep;                     // value heads h0 .. h0+rep-1 (qwen.c:331, 335)
    const int key_dim = kh * KD, vdim = vh * VD, conv_dim = 2 * key_dim + vdim;
    const size_t tok = (size_t)l * args.B + b;

    const int tid = threadIdx.x;
    const int c4 = tid % C4, rg = tid / C4;
    const int lane = tid % OMH_WAVE, wave = tid / OMH_WAVE;
    float *S0 = Sl + ((size_t)seq * vh + h0) * (KD * VD);

    __shared__ __align__(16) float s_q[KD], s_k[KD], s_v[REPMAX * VD], s_z[REPMAX * VD];
    __shared__ float s_gam[REPMAX], s_beta[REPMAX];
    __shared__ float4 s_red[2][NW][2][C4];

    // The first two value heads' state tiles (REPMAX >= 2 means rep >= 2)
    // are requested before anything else: starting every workgroup's HBM
    // stream at once beats having the prologue's small scattered reads
    // (which then wait behind the tiles) ready early.  On MI355X, 30 layers
    // x 1 sequence: 23.8 us per launch in this order; 26.3 us with the
    // prologue's inputs requested between the two tiles (so the first head
    // could start earlier) and 27.3 us with them requested first.
    float4 sa[Sh::RPT], sb[Sh::RPT];
    load_head<KD, VD>(sa, S0, rg, c4);
    if constexpr (REPMAX > 1) load_head<KD, VD>(sb, S0 + KD * VD, rg, c4);
    __builtin_amdgcn_sched_barrier(0);           // nothing (the phase load included) moves above the tile requests

    // (1) Prologue: the conv channels of key head hk (q, k) and of its
    // value heads (v), z of the value heads, the gate inputs.  This
    // workgroup owns all of these channels and appends them to the ring.
    const int ph = L.phase[L.epoch * L.max_seqs + seq];
    const float *qkv = args.qkv + tok * args.ld_qkv;
    const int nch = 2 * KD + rep * VD;
    ConvIn<NIT> cin;
    cin.load([&](int c) {
                 return c < KD ? hk * KD + c
                               : (c < 2 * KD ? key_dim + hk * KD + (c - KD) : 2 * key_dim + h0 * VD + (c - 2 * KD));
             },
             nch, tid, TPB, qkv, L.conv_w, L.conv_st, conv_dim, seq, ph, K);
    const float *zrow = args.z + tok * args.ld_z + (size_t)h0 * VD;
    float zin[NZ];
#pragma unroll
    for (int it = 0; it < NZ; it++) {
        const int c = tid + it * TPB;
        zin[it] = zrow[c < rep * VD ? c : 0];
    }
    const int gh = h0 + (tid < rep ? tid : rep - 1);
    const float ga = args.a[tok * args.ld_ab + gh], gb = args.b[tok * args.ld_ab + gh];
    const float galog = L.A_log[gh], gdt = L.dt_bias[gh];
    const float4 gn = *reinterpret_cast<const float4 *>(L.gnorm + c4 * 4);

#pragma unroll
    for (int it = 0; it < NIT; it++) {
        if (cin.gch[it] < 0) continue;
        const int c = tid + it * TPB;
        const float y = cin.template conv<false>(it, K);
        if (c < KD) s_q[c] = y;
        else if (c < 2 * KD) s_k[c - KD] = y;
        else s_v[c - 2 * KD] = y;
        cin.append(it, L.conv_st, conv_dim, seq, ph);
    }
#pragma unroll
    for (int it = 0; it < NZ; it++) {
        const int c = tid + it * TPB;
        if (c < rep * VD) s_z[c] = zin[it];
    }
    if (tid < rep) {
        // gates (qwen.c:337-338)
        const float g = -expf(galog) * omh_softplus(ga + gdt);
        s_gam[tid] = expf(g);
        s_beta[tid] = omh_sigmoid(gb);
    }
    omh_lds_barrier();
    HeadCoef hc;
    qk_factors<KD, false>(s_q, s_k, lane, hc.rq, hc.rk, hc.kq);

    // (3)+(4) value heads in order; the next head's state is in flight while
    // the current one is reduced and written back.  Heads alternate between
    // the two reduction buffers, so a wave that runs ahead into the next
    // head never overwrites sums another wave is still reading.
    float *core = args.core + tok * vdim + (size_t)h0 * VD;
    const PlaneOut po{args.xb, args.xb_T, vdim, args.xb_i8};
    for (int j = 0; j < rep; j += 2) {
        hc.gam = s_gam[j];
        hc.beta = s_beta[j];
        paired_head<KD, VD>(sa, S0 + (size_t)j * KD * VD, core + j * VD, s_q, s_k, s_v + j * VD, s_z + j * VD, hc,
                            gn, args.eps, s_red[0], wave, lane, c4, rg, po, args.xb_t0 + b, (h0 + j) * VD);
        if (j + 2 < rep) load_head<KD, VD>(sa, S0 + (size_t)(j + 2) * KD * VD, rg, c4);
        if (REPMAX > 1 && j + 1 < rep) {
            hc.gam = s_gam[j + 1];
            hc.beta = s_beta[j + 1];
            paired_head<KD, VD>(sb, S0 + (size_t)(j + 1) * KD * VD, core + (j + 1) * VD, s_q, s_k,
                                s_v + (j + 1) * VD, s_z + (j + 1) * VD, hc, gn, args.eps, s_red[1], wave, lane,
                                c4, rg, po, args.xb_t0 + b, (h0 + j + 1) * VD);
            if (j + 3 < rep) load_head<KD, VD>(sb, S0 + (size_t)(j + 3) * KD * VD, rg, c4);
        }
    }
    advance_phase(L, args.b0, args.B, seq, hk == 0, hk == 0 && b == 0, ph, tid, TPB);
}

// ------------------------------------------------------------- sliced kernel
template <int KD, int VD, int NCS>
__global__ __launch_bounds__((TileShape<KD, VD / NCS, kSliceMaxT>::TPB))
void gdn_decode_core_kernel(const DecodeArgs args) {
    using Sh = TileShape<KD, VD / NCS, kSliceMaxT>;
    constexpr int TPB = Sh::TPB, CW = VD / NCS, C4 = Sh::C4, RG = Sh::RG, RPT = Sh::RPT, NW = Sh::NW;
    static_assert(NCS <= kMaxSlices && VD / 4 <= TPB, "norm epilogue layout");

    const int cs = blockIdx.x % NCS;             // column slice
    const int h = blockIdx.x / NCS;              // value head
    const int b = blockIdx.y;                    // token row of the launch
    const int seq = args.b0 + b;                 // sequence (state slot)
    const int l = blockIdx.z;                    // layer slot
    const LayerPtrs &L = args.L[l];
    float *const Sl = L.S;
    const int kh = args.kh, vh = args.vh, K = args.K, rep = args.rep;
    // The argument block's other 64-byte lines (the input pointers', the
    // layer's epoch) are requested in the same batch: read where first used,
    // each line cost one more dependent round trip before the first load.
    const float *const qkv_arg = args.qkv;
    const int epoch = L.epoch, max_seqs = L.max_seqs;
    __builtin_amdgcn_sched_barrier(0);           // the state pointer is requested with the counts
    const int hk = h / rep;                      // key head of value head h (qwen.c:331, 335)
    const int key_dim = kh * KD, vdim = vh * VD, conv_dim = 2 * key_dim + vdim;
    const size_t tok = (size_t)l * args.B + b;
    const int col0 = cs * CW;

    const int tid = threadIdx.x;
    const int c4 = tid % C4, rg = tid / C4;
    const int lane = tid % OMH_WAVE, wave = tid / OMH_WAVE;
    float *Sp = Sl + ((size_t)seq * vh + h) * (KD * VD) + col0;

    __shared__ __align__(16) float s_q[KD], s_k[KD], s_v[CW];
    __shared__ float s_gam, s_beta;
    __shared__ float4 s_red[NW][2][C4];
    __shared__ int s_last;

    // (1) Every prologue request goes out before any of them is waited
    // for: the q/k channels of key head hk (recomputed by every workgroup of
    // the key head, appended by its first one) and this slice's value
    // channels with all their ring slots (ConvIn ALL: the phase only picks
    // among them afterwards), z and gnorm, then the gate inputs and the ring
    // phase (wave-uniform loads, issued after the vector requests so that
    // none of those waits for them), then the state slice.  With the ring
    // loads behind the phase and the gate loads behind both, one layer at
    // B = 1 waited for two more dependent round trips.
    constexpr int NIT = (2 * KD + CW + TPB - 1) / TPB;
    const float *qkv = qkv_arg + tok * args.ld_qkv;
    ConvIn<NIT, true> cin;
    cin.load([&](int c) {
                 return c < KD ? hk * KD + c
                               : (c < 2 * KD ? key_dim + hk * KD + (c - KD) : 2 * key_dim + h * VD + col0 + (c - 2 * KD));
             },
             2 * KD + CW, tid, TPB, qkv, L.conv_w, L.conv_st, conv_dim, seq, 0, K);
    const int t4 = tid < VD / 4 ? tid : 0;
    // z and gnorm of the columns this thread gates: the head's columns 4 t4
    // (norm here), or the slice's own columns (1 / rms left to the consumer)
    const int zc = args.ssq_out ? col0 + 4 * c4 : 4 * t4;
    const float4 zz = *reinterpret_cast<const float4 *>(args.z + tok * args.ld_z + (size_t)h * VD + zc);
    const float4 gn = *reinterpret_cast<const float4 *>(L.gnorm + zc);
    __builtin_amdgcn_sched_barrier(0);
    const float ga = args.a[tok * args.ld_ab + h], gb = args.b[tok * args.ld_ab + h];
    const float galog = L.A_log[h], gdt = L.dt_bias[h];
    const int ph = L.phase[epoch * max_seqs + seq];

    float4 s[RPT];
    const __amdgpu_buffer_rsrc_t rs = omh_rsrc(Sp, (KD * VD - col0) * 4);
#pragma unroll
    for (int m = 0; m < RPT; m++) s[m] = omh_ld_stream_buf(rs, ((rg + RG * m) * VD + c4 * 4) * 4);
    __builtin_amdgcn_sched_barrier(0);           // keep prologue arithmetic after the state requests
    cin.pick(ph, K);

    const bool own_qk = (h % rep == 0) && cs == 0;
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        if (cin.gch[it] < 0) continue;
        const int c = tid + it * TPB;
        const float y = cin.template conv<true>(it, K);
        bool own = true;
        if (c < KD) { s_q[c] = y; own = own_qk; }
        else if (c < 2 * KD) { s_k[c - KD] = y; own = own_qk; }
        else s_v[c - 2 * KD] = y;
        if (own) cin.append(it, L.conv_st, conv_dim, seq, ph);
    }
    if (tid == TPB - OMH_WAVE) {
        // gates (qwen.c:337-338), on the last wave: it converts the fewest
        // channels above, so this serial chain overlaps the others' work
        const float g = -expf(galog) * omh_softplus(ga + gdt);
        s_gam = expf(g);
        s_beta = omh_sigmoid(gb);
    }
    omh_lds_barrier();
    HeadCoef hc;
    qk_factors<KD, true>(s_q, s_k, lane, hc.rq, hc.rk, hc.kq);
    hc.gam = s_gam;
    hc.beta = s_beta;

    // (3) delta rule on this slice of value head h (qwen.c:339-352)
    const float4 vv = *reinterpret_cast<const float4 *>(&s_v[c4 * 4]);
    const float4 o = delta_rule<KD, VD, RG, RPT, C4, NW>(s, Sp, s_q, s_k, vv, hc, s_red, wave, lane, c4, rg);
    advance_phase(L, args.b0, args.B, seq, h == 0 && cs == 0, h == 0 && cs == 0 && b == 0, ph, tid, TPB);

    // (4) gated RMSNorm over the head's vd columns (qwen.c:353-357)
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = omh_lane_sum_below<C4>(ss);              // this slice's sum of squares
    float *core = args.core + tok * vdim + (size_t)h * VD;
    if constexpr (NCS == 1) {
        if (rg == 0) {
            const float rn = rsqrtf(ss / (float)VD + args.eps);
            const float4 y = gated<true>(o, rn, gn, zz);
            *reinterpret_cast<float4 *>(core + c4 * 4) = y;
            if constexpr (VD % 64 == 0)
                if (args.xb) write_x(PlaneOut{args.xb, args.xb_T, vdim, args.xb_i8}, args.xb_t0 + b, h * VD + c4 * 4, c4, y);
        }
    } else if (args.ssq_out) {
        // Deferred norm: this slice's o * gnorm * silu(z) and its sum of
        // squares of o; the next launch (out_proj's GEMV) applies 1 / rms as
        // it loads them, so no slice waits for another.
        if (rg == 0) *reinterpret_cast<float4 *>(core + col0 + c4 * 4) = gated<true>(o, 1.f, gn, zz);
        if (tid == 0) args.ssq_out[(tok * vh + h) * NCS + cs] = ss;
    } else {
        // Cross-slice exchange with device-coherent (agent-scope) relaxed
        // atomics only: they bypass the per-XCD L2s, so no L2 write-back is
        // needed (an agent-scope fence would write back the whole L2).  Each
        // thread waits for its own stores to complete before the workgroup
        // barrier, and only then is the arrival counted.
        const size_t hb = (size_t)seq * vh + h;
        if (rg == 0) {
            float *dst = L.o_raw + hb * VD + col0 + c4 * 4;
            __hip_atomic_store(dst + 0, o.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + 1, o.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + 2, o.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + 3, o.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid == 0) __hip_atomic_store(L.ssq + hb * kMaxSlices + cs, ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);           // this thread's stores are complete
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(L.cnt + hb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == NCS - 1;
        __syncthreads();
        if (s_last) {
            if (tid < VD / 4) {
                float tot = 0.f;
#pragma unroll
                for (int k = 0; k < NCS; k++)
                    tot += __hip_atomic_load(L.ssq + hb * kMaxSlices + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float rn = rsqrtf(tot / (float)VD + args.eps);
                const float *src = L.o_raw + hb * VD + tid * 4;
                float4 oo;
                oo.x = __hip_atomic_load(src + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *reinterpret_cast<float4 *>(core + tid * 4) = gated<true>(oo, rn, gn, zz);
            }
            if (tid == 0) __hip_atomic_store(L.cnt + hb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int KD, int VD, int NCS>
hipError_t launch_sliced(const DecodeArgs &a, hipStream_t st) {
    dim3 grid(a.vh * NCS, a.B, a.nl);
    hipLaunchKernelGGL((gdn_decode_core_kernel<KD, VD, NCS>), grid, dim3(TileShape<KD, VD / NCS, kSliceMaxT>::TPB), 0,
                       st, a);
    return hipGetLastError();
}

template <int KD, int VD>
hipError_t launch_kd_vd(const DecodeArgs &a, int variant, hipStream_t st) {
    switch (variant) {
        case kDecodePaired: {
            const int rep = a.vh / a.kh;
            const dim3 grid(a.kh, a.B, a.nl), block(PairShape<KD, VD>::TPB);
            if (rep == 1) hipLaunchKernelGGL((gdn_decode_paired_kernel<KD, VD, 1>), grid, block, 0, st, a);
            else if (rep == 2) hipLaunchKernelGGL((gdn_decode_paired_kernel<KD, VD, 2>), grid, block, 0, st, a);
            else if (rep <= 4) hipLaunchKernelGGL((gdn_decode_paired_kernel<KD, VD, 4>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((gdn_decode_paired_kernel<KD, VD, kMaxRep>), grid, block, 0, st, a);
            return hipGetLastError();
        }
        case 1: if constexpr (slice_valid(KD, VD, 1)) return launch_sliced<KD, VD, 1>(a, st); break;
        case 2: if constexpr (slice_valid(KD, VD, 2)) return launch_sliced<KD, VD, 2>(a, st); break;
        case 4: if constexpr (slice_valid(KD, VD, 4)) return launch_sliced<KD, VD, 4>(a, st); break;
        case 8: if constexpr (slice_valid(KD, VD, 8)) return launch_sliced<KD, VD, 8>(a, st); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

// Launch-size rule: the paired kernel once the launch has enough key-head
// workgroups to cover the chip (30 layers x 1 sequence: 24.8 us paired vs
// 28.4 us one workgroup per head on MI355X); below that one workgroup per
// value head.  Column slices do not pay on MI355X even for one layer at
// B = 1 (7.4 us at NCS = 1, 8.1 / 8.2 / 9.0 us at NCS = 2 / 4 / 8): the
// step is latency-bound there and the cross-slice exchange adds a round
// trip.  They stay available through the variant argument.
int choose_variant(const DecodeArgs &a, int kd, int vd) {
    (void)kd; (void)vd;
    const long pair_wgs = (long)a.nl * a.B * a.kh;
    const int rep = a.vh / a.kh;
    if (pair_wgs >= 256 && rep <= kMaxRep) return kDecodePaired;
    return 1;
}

}  // namespace

bool decode_core_supported(int kd, int vd, int rep, int K) {
    if (rep < 1 || K < 2 || K > kConvRing) return false;
    return (kd == vd && (kd == 16 || kd == 32 || kd == 64 || kd == 128)) || (kd == 32 && vd == 16);
}

// Resident workgroups of the paired kernel per round: two per CU (its
// registers allow two waves per SIMD), 256 CUs.
constexpr long kPairedRound = 512;

int decode_seqs_per_launch(int kd, int vd, int kh, int vh, int nl, int B, int variant) {
    if (nl != 1 || kh < 1) return B;
    DecodeArgs probe{};
    probe.nl = nl;
    probe.B = B;
    probe.kh = kh;
    probe.vh = vh;
    if ((variant == 0 ? choose_variant(probe, kd, vd) : variant) != kDecodePaired) return B;
    const long wgs = (long)kh * B;
    if (wgs <= kPairedRound) return B;
    const int chunks = (int)((wgs + kPairedRound - 1) / kPairedRound);
    return (B + chunks - 1) / chunks;
}

bool decode_planes_supported(int vd, int variant, bool i8) {
    return vd % (i8 ? kI8Blk : 64) == 0 && (variant == 0 || variant == kDecodePaired || variant == 1);
}

// Column slices for a deferred-norm launch (one layer, up to 4 tokens): 4
// per value head, no exchange between them.  35B shape, engine-order chain
// of 30 whole int8 layers at B = 1, MI355X: 17.8 us per layer with 4 slices
// and the 1 / rms in out_proj's GEMV (core 5.8 us), 18.2 us with one
// workgroup per value head and the norm in the core (core 6.5 us); timing
// copies without any norm put 2 and 8 slices behind 4.
int decode_deferred_slices(int kd, int vd) {
    return slice_valid(kd, vd, 4) && vd % 16 == 0 ? 4 : 0;
}

hipError_t launch_decode_core(const DecodeArgs &a, int kd, int vd, int variant, hipStream_t st) {
    if (!decode_core_supported(kd, vd, a.vh / a.kh, a.K)) return hipErrorInvalidValue;
    if (a.ssq_out && (a.nl != 1 || variant != 4 || a.xb)) return hipErrorInvalidValue;
    if (a.rep != a.vh / a.kh) return hipErrorInvalidValue;
    if (a.xb && (a.nl != 1 || !decode_planes_supported(vd, variant, a.xb_i8))) return hipErrorInvalidValue;
    if (variant == 0) variant = choose_variant(a, kd, vd);
    if (variant == kDecodePaired && a.vh / a.kh > kMaxRep) return hipErrorInvalidValue;
    if (kd == 16 && vd == 16) return launch_kd_vd<16, 16>(a, variant, st);
    if (kd == 32 && vd == 32) return launch_kd_vd<32, 32>(a, variant, st);
    if (kd == 64 && vd == 64) return launch_kd_vd<64, 64>(a, variant, st);
    if (kd == 128 && vd == 128) return launch_kd_vd<128, 128>(a, variant, st);
    if (kd == 32 && vd == 16) return launch_kd_vd<32, 16>(a, variant, st);
    return hipErrorInvalidValue;
}

// State snapshot / rollback: blockIdx.y = layer, one float4 of the S block
// and of the conv ring per thread (HBM-bound, 2 x 2.2 MB per layer at the
// 35B shape), and the ring phase by the first thread.  Nontemporal loads and
// stores: 30 layers of the 35B shape, 536 MB rotated, MI355X: 22.9 us
// against 26.1 us with plain ones.
__global__ __launch_bounds__(256) void state_copy_kernel(const StateCopyArgs c) {
    const int l = blockIdx.y;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;   // one float4 of S and of the ring
    if (i < c.n4) omh_st_stream(c.S_dst[l] + 4 * i, omh_ld_stream(c.S_src[l] + 4 * i));
    if (i < c.r4) omh_st_stream(c.R_dst[l] + 4 * i, omh_ld_stream(c.R_src[l] + 4 * i));
    if (i == 0) *c.P_dst[l] = *c.P_src[l];
}

hipError_t launch_state_copy(const StateCopyArgs &c, hipStream_t st) {
    if (c.nl < 1 || c.nl > kMaxDecodeLayers) return hipErrorInvalidValue;
    const size_t per = c.n4 > c.r4 ? c.n4 : c.r4;
    const unsigned gx = (unsigned)((per + 255) / 256);
    hipLaunchKernelGGL(state_copy_kernel, dim3(gx, (unsigned)c.nl), dim3(256), 0, st, c);
    return hipGetLastError();
}

}  // namespace omh
