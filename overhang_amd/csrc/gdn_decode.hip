// gdn_decode.hip — one-token GDN core for many (layer, sequence) slots.
//
// Fuses, for one token, the three decode-side stages of the layer core
// (overhang engines/qwen.c:307-358):
//   (1) causal conv1d update (kernel K) + SiLU, per-head q/k L2 norm and q
//       scale, gates g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
//   (3) the gated delta-rule update of the fp32 state S[kd][vd] of each
//       value head:  S <- gamma S;  kv = S^T k;  delta = beta (v - kv);
//       S <- S + k delta^T;  o = S^T q;
//   (4) the gated RMSNorm  o * rsqrt(mean(o^2) + eps) * gnorm * silu(z).
//
// One workgroup owns one key head of one (layer, sequence) slot together
// with the REP value heads that share it (value head h uses key head
// h / REP, qwen.c:331, 335).  Every conv channel then has exactly one owner,
// so the conv history is updated in place with no cross-workgroup ordering,
// and each value head's state is read once and written once, straight from
// registers: the kernel is bound by HBM at 2*kd*vd*4 bytes per value head.
//
// Thread layout per value head: TPH threads, each holding RPT rows x 4
// adjacent columns (a float4) of S.  A wavefront's loads cover whole
// consecutive rows, so every load/store instruction moves contiguous 1 KiB
// (kd = vd = 128).  Column sums over rows (S^T k, S^T q) are butterfly
// reductions across the row groups of a wave, then across the head's waves
// through LDS.
#include "omh_device.h"
#include "omh_internal.h"

namespace omh {
namespace {

template <int KD, int VD>
struct DecodeShape {
    static constexpr int C4 = VD / 4;                       // float4 columns per row
    static constexpr int TPH_RAW = KD * C4 / 8;             // aim for ~8 float4 per thread
    static constexpr int TPH = TPH_RAW < 64 ? 64 : (TPH_RAW > 256 ? 256 : TPH_RAW);
    static constexpr int RG = TPH / C4;                     // row groups
    static constexpr int RPT = KD / RG;                     // rows per thread
    static constexpr int WPH = TPH / OMH_WAVE;              // waves per value head
    static_assert(VD % 4 == 0 && C4 <= OMH_WAVE && TPH % C4 == 0, "vd layout");
    static_assert(RG >= 1 && KD % RG == 0 && RPT >= 1, "kd layout");
    static_assert(TPH % OMH_WAVE == 0, "whole waves per head");
};

// Sum a float4 over the row groups of one value head (every thread of the
// head receives the column sums of its 4 columns).
template <int KD, int VD>
__device__ __forceinline__ float4 head_colsum(float4 x, float4 (*red)[DecodeShape<KD, VD>::C4],
                                              int wave_in_head, int lane, int c4) {
    using Sh = DecodeShape<KD, VD>;
    x.x = omh_xor_sum_from<Sh::C4>(x.x);
    x.y = omh_xor_sum_from<Sh::C4>(x.y);
    x.z = omh_xor_sum_from<Sh::C4>(x.z);
    x.w = omh_xor_sum_from<Sh::C4>(x.w);
    if constexpr (Sh::WPH > 1) {
        if (lane < Sh::C4) red[wave_in_head][c4] = x;
        omh_lds_barrier();
        x = red[0][c4];
#pragma unroll
        for (int w = 1; w < Sh::WPH; w++) {
            float4 y = red[w][c4];
            x.x += y.x; x.y += y.y; x.z += y.z; x.w += y.w;
        }
    }
    return x;
}

template <int KD, int VD, int REP>
__global__ __launch_bounds__((REP * DecodeShape<KD, VD>::TPH))
void gdn_decode_core_kernel(const DecodeArgs args) {
    using Sh = DecodeShape<KD, VD>;
    constexpr int TPH = Sh::TPH, C4 = Sh::C4, RG = Sh::RG, RPT = Sh::RPT, WPH = Sh::WPH;
    constexpr int NT = REP * TPH;
    constexpr int CH = 2 * KD + REP * VD;        // conv channels owned by this workgroup

    const int jk = blockIdx.x;                   // key head
    const int b = blockIdx.y;                    // sequence
    const int l = blockIdx.z;                    // layer slot
    const LayerPtrs &L = args.L[l];
    const int kh = args.kh, vh = args.vh, K = args.K;
    const int key_dim = kh * KD, vdim = vh * VD, conv_dim = 2 * key_dim + vdim;
    const size_t tok = (size_t)l * args.B + b;
    const float *qkv = args.qkv + tok * args.ld_qkv;

    __shared__ float s_q[KD], s_k[KD];
    __shared__ float s_v[REP * VD];
    __shared__ float s_gam[REP], s_beta[REP];
    __shared__ float4 s_red1[REP][WPH][C4];
    __shared__ float4 s_red2[REP][WPH][C4];

    const int tid = threadIdx.x;
    const int r = tid / TPH, lt = tid % TPH;
    const int c4 = lt % C4, rg = lt / C4;
    const int lane = tid % OMH_WAVE, wih = lt / OMH_WAVE;
    const int h = jk * REP + r;
    float *Sp = L.S + ((size_t)b * vh + h) * (KD * VD);

    // Issue the state loads first: nothing before the delta rule depends on
    // them, so their HBM latency overlaps the conv/norm prologue below (the
    // barriers there order LDS only and leave these loads in flight).
    float4 s[RPT];
#pragma unroll
    for (int m = 0; m < RPT; m++)
        s[m] = omh_ld_stream(Sp + (size_t)(rg + RG * m) * VD + c4 * 4);
    float4 zz = f4_zero(), gn = f4_zero();
    if (rg == 0) {
        zz = *reinterpret_cast<const float4 *>(args.z + tok * args.ld_z + (size_t)h * VD + c4 * 4);
        gn = *reinterpret_cast<const float4 *>(L.gnorm + c4 * 4);
    }

    // (1) conv update + SiLU for the q/k channels of key head jk and the v
    // channels of its REP value heads (op order as qwen.c:311-319).
    float *hist_base = L.conv_st + (size_t)b * conv_dim * (K - 1);
    for (int c = tid; c < CH; c += NT) {
        int gch;
        float *dst;
        if (c < KD) { gch = jk * KD + c; dst = &s_q[c]; }
        else if (c < 2 * KD) { gch = key_dim + jk * KD + (c - KD); dst = &s_k[c - KD]; }
        else { gch = 2 * key_dim + jk * REP * VD + (c - 2 * KD); dst = &s_v[c - 2 * KD]; }
        const float *w = L.conv_w + (size_t)gch * K;
        float *h = hist_base + (size_t)gch * (K - 1);
        const float x = qkv[gch];
        float acc = 0.f;
        for (int j = 0; j < K - 1; j++) acc += w[j] * h[j];
        acc += w[K - 1] * x;
        for (int j = 0; j < K - 2; j++) h[j] = h[j + 1];
        h[K - 2] = x;
        *dst = omh_silu(acc);
    }
    // gates (qwen.c:337-338)
    if (tid < REP) {
        const int h = jk * REP + tid;
        const float g = -expf(L.A_log[h]) * omh_softplus(args.a[tok * args.ld_ab + h] + L.dt_bias[h]);
        s_gam[tid] = expf(g);
        s_beta[tid] = omh_sigmoid(args.b[tok * args.ld_ab + h]);
    }
    omh_lds_barrier();
    // L2 norm of q and k (eps 1e-6), then q *= kd^-1/2 (qwen.c:153-157, 326-329)
    if (tid < OMH_WAVE) {
        float sq = 0.f, sk = 0.f;
        for (int i = tid; i < KD; i += OMH_WAVE) { sq += s_q[i] * s_q[i]; sk += s_k[i] * s_k[i]; }
        sq = omh_xor_sum_below<OMH_WAVE>(sq);
        sk = omh_xor_sum_below<OMH_WAVE>(sk);
        const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f);
        const float scale = 1.f / sqrtf((float)KD);
        for (int i = tid; i < KD; i += OMH_WAVE) { s_q[i] = (s_q[i] * rq) * scale; s_k[i] *= rk; }
    }
    omh_lds_barrier();

    // (3) delta rule on value head h (qwen.c:339-352)
    const float gam = s_gam[r], beta = s_beta[r];
    float4 kv = f4_zero();
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        s[m] = f4_scale(s[m], gam);
        kv = f4_fma(s[m], s_k[rg + RG * m], kv);
    }
    kv = head_colsum<KD, VD>(kv, s_red1[r], wih, lane, c4);

    const float4 vv = *reinterpret_cast<const float4 *>(&s_v[r * VD + c4 * 4]);
    const float4 delta = f4_scale(f4_sub(vv, kv), beta);
    float4 o = f4_zero();
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        const int i = rg + RG * m;
        s[m] = f4_fma(delta, s_k[i], s[m]);
        o = f4_fma(s[m], s_q[i], o);
        omh_st_stream(Sp + (size_t)i * VD + c4 * 4, s[m]);
    }
    o = head_colsum<KD, VD>(o, s_red2[r], wih, lane, c4);

    // (4) gated RMSNorm (qwen.c:353-357): the C4 lanes of a row group hold
    // the whole head row.
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = omh_xor_sum_below<C4>(ss);
    if (rg == 0) {
        const float rn = 1.f / sqrtf(ss / (float)VD + args.eps);
        const size_t off = tok * vdim + (size_t)h * VD + c4 * 4;
        float4 y;
        y.x = o.x * rn * gn.x * omh_silu(zz.x);
        y.y = o.y * rn * gn.y * omh_silu(zz.y);
        y.z = o.z * rn * gn.z * omh_silu(zz.z);
        y.w = o.w * rn * gn.w * omh_silu(zz.w);
        *reinterpret_cast<float4 *>(args.core + off) = y;
    }
}

template <int KD, int VD, int REP>
hipError_t launch_one(const DecodeArgs &a, hipStream_t st) {
    dim3 grid(a.kh, a.B, a.nl);
    dim3 block(REP * DecodeShape<KD, VD>::TPH);
    hipLaunchKernelGGL((gdn_decode_core_kernel<KD, VD, REP>), grid, block, 0, st, a);
    return hipGetLastError();
}

template <int KD, int VD>
hipError_t launch_rep(const DecodeArgs &a, int rep, hipStream_t st) {
    switch (rep) {
        case 1: return launch_one<KD, VD, 1>(a, st);
        case 2: return launch_one<KD, VD, 2>(a, st);
        case 3: return launch_one<KD, VD, 3>(a, st);
        case 4: return launch_one<KD, VD, 4>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool decode_core_supported(int kd, int vd, int rep) {
    if (rep < 1 || rep > 4) return false;
    return (kd == vd && (kd == 16 || kd == 32 || kd == 64 || kd == 128)) || (kd == 32 && vd == 16);
}

hipError_t launch_decode_core(const DecodeArgs &a, int kd, int vd, hipStream_t st) {
    const int rep = a.vh / a.kh;
    if (!decode_core_supported(kd, vd, rep)) return hipErrorInvalidValue;
    if (kd == 16 && vd == 16) return launch_rep<16, 16>(a, rep, st);
    if (kd == 32 && vd == 32) return launch_rep<32, 32>(a, rep, st);
    if (kd == 64 && vd == 64) return launch_rep<64, 64>(a, rep, st);
    if (kd == 128 && vd == 128) return launch_rep<128, 128>(a, rep, st);
    if (kd == 32 && vd == 16) return launch_rep<32, 16>(a, rep, st);
    return hipErrorInvalidValue;
}

}  // namespace omh
