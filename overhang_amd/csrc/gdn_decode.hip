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
// The kernel is bound by HBM: each value head's state is read once and
// written once (2*kd*vd*4 bytes), with streaming (nontemporal) accesses.
// The delta rule couples only the rows of one column (kv, delta and o of
// column j involve S[:, j] alone), so a value head may be split into NCS
// column slices, one workgroup each (a step of B sequences x nl layers runs
// nl*B*vh*NCS workgroups); NCS = 1 is the default, see default_ncs().
//
// Each workgroup recomputes the conv + L2 norm of its key head (q and k are
// needed whole) and the conv of its own value columns.  Conv history lives
// in a 4-slot ring per channel (omh_internal.h): readers use the K-1 history
// slots, the single owner of a channel appends the new input into the free
// slot, so no workgroup ever reads what another writes in the same launch.
// The gated RMSNorm needs the whole row of o: with NCS > 1 each slice
// publishes its raw o and its partial sum of squares (device-coherent
// atomic stores), and the last slice of the head to arrive (arrival
// counter) applies the norm to all vd columns, summing the partials in
// slice order, so the result does not depend on arrival order.
//
// Thread layout: TPB threads hold RPT rows x 4 adjacent columns (a float4)
// of the slice; a wavefront's loads cover whole consecutive row segments.
// Column sums over rows are butterflies across the row groups of a wave,
// then across waves through LDS.
#include "omh_device.h"
#include "omh_internal.h"

namespace omh {
namespace {

template <int KD, int VD, int NCS>
struct DecShape {
    static constexpr int CW = VD / NCS;                     // columns per workgroup
    static constexpr int C4 = CW / 4;                       // float4 columns per row
    static constexpr int TPB_RAW = KD * C4 / 4;             // aim for 4 float4 per thread
    static constexpr int TPB = TPB_RAW < 64 ? 64 : (TPB_RAW > 256 ? 256 : TPB_RAW);
    static constexpr int RG = TPB / C4;                     // row groups
    static constexpr int RPT = KD / RG;                     // rows per thread
    static constexpr int NW = TPB / OMH_WAVE;
    static_assert(VD % NCS == 0 && CW % 4 == 0 && C4 >= 1 && C4 <= OMH_WAVE, "slice layout");
    static_assert((C4 & (C4 - 1)) == 0 && TPB % C4 == 0, "slice layout");
    static_assert(RG >= 1 && KD % RG == 0 && RPT >= 1, "row layout");
    static_assert(NCS <= kMaxSlices && VD / 4 <= TPB, "norm epilogue layout");
};

// Whether DecShape<KD, VD, NCS> is a valid layout (checked before use).
constexpr bool dec_valid_rt(int KD, int VD, int NCS) {
    if (NCS < 1 || VD % NCS != 0 || (VD / NCS) % 4 != 0 || NCS > kMaxSlices) return false;
    const int c4 = VD / NCS / 4;
    if (c4 < 1 || c4 > OMH_WAVE || (c4 & (c4 - 1)) != 0) return false;
    const int raw = KD * c4 / 4;
    const int tpb = raw < 64 ? 64 : (raw > 256 ? 256 : raw);
    const int rg = tpb / c4;
    return tpb % c4 == 0 && rg <= KD && KD % rg == 0 && VD / 4 <= tpb;
}
template <int KD, int VD, int NCS>
constexpr bool dec_valid() { return dec_valid_rt(KD, VD, NCS); }

// Sum a float4 over the row groups of the workgroup.
template <int C4, int NW>
__device__ __forceinline__ float4 colsum(float4 x, float4 (*red)[C4], int wave, int lane, int c4) {
    x.x = omh_xor_sum_from<C4>(x.x);
    x.y = omh_xor_sum_from<C4>(x.y);
    x.z = omh_xor_sum_from<C4>(x.z);
    x.w = omh_xor_sum_from<C4>(x.w);
    if constexpr (NW > 1) {
        if (lane < C4) red[wave][c4] = x;
        omh_lds_barrier();
        x = red[0][c4];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            const float4 y = red[w][c4];
            x.x += y.x; x.y += y.y; x.z += y.z; x.w += y.w;
        }
    }
    return x;
}

__device__ __forceinline__ float4 gated(float4 o, float rn, float4 gn, float4 zz) {
    float4 y;
    y.x = o.x * rn * gn.x * omh_silu(zz.x);
    y.y = o.y * rn * gn.y * omh_silu(zz.y);
    y.z = o.z * rn * gn.z * omh_silu(zz.z);
    y.w = o.w * rn * gn.w * omh_silu(zz.w);
    return y;
}

template <int KD, int VD, int NCS>
__global__ __launch_bounds__((DecShape<KD, VD, NCS>::TPB))
void gdn_decode_core_kernel(const DecodeArgs args) {
    using Sh = DecShape<KD, VD, NCS>;
    constexpr int TPB = Sh::TPB, CW = Sh::CW, C4 = Sh::C4, RG = Sh::RG, RPT = Sh::RPT, NW = Sh::NW;

    const int cs = blockIdx.x % NCS;             // column slice
    const int h = blockIdx.x / NCS;              // value head
    const int b = blockIdx.y;                    // sequence
    const int l = blockIdx.z;                    // layer slot
    const LayerPtrs &L = args.L[l];
    const int kh = args.kh, vh = args.vh, K = args.K;
    const int rep = vh / kh, hk = h / rep;       // key head of value head h (qwen.c:331, 335)
    const int key_dim = kh * KD, vdim = vh * VD, conv_dim = 2 * key_dim + vdim;
    const size_t tok = (size_t)l * args.B + b;
    const int col0 = cs * CW;

    const int tid = threadIdx.x;
    const int c4 = tid % C4, rg = tid / C4;
    const int lane = tid % OMH_WAVE, wave = tid / OMH_WAVE;
    float *Sp = L.S + ((size_t)b * vh + h) * (KD * VD) + col0;

    __shared__ float s_q[KD], s_k[KD], s_v[CW];
    __shared__ float s_gam, s_beta;
    __shared__ float4 s_red1[NW][C4], s_red2[NW][C4];
    __shared__ int s_last;

    // State loads first: nothing before the delta rule depends on them, so
    // their latency overlaps the prologue (whose barriers order LDS only).
    float4 s[RPT];
#pragma unroll
    for (int m = 0; m < RPT; m++) s[m] = omh_ld_stream(Sp + (size_t)(rg + RG * m) * VD + c4 * 4);
    float4 zz = f4_zero(), gn = f4_zero();
    if (tid < VD / 4) {
        zz = *reinterpret_cast<const float4 *>(args.z + tok * args.ld_z + (size_t)h * VD + tid * 4);
        gn = *reinterpret_cast<const float4 *>(L.gnorm + tid * 4);
    }

    // (1) conv + SiLU (op order as qwen.c:311-319) for the q/k channels of
    // key head hk and this slice's value channels.
    const int ph = L.phase[L.epoch * L.max_seqs + b];
    const float *qkv = args.qkv + tok * args.ld_qkv;
    float *ring = L.conv_st + (size_t)b * conv_dim * kConvRing;
    const bool own_qk = (h % rep == 0) && cs == 0;
    for (int c = tid; c < 2 * KD + CW; c += TPB) {
        int gch;
        float *dst;
        bool own;
        if (c < KD) { gch = hk * KD + c; dst = &s_q[c]; own = own_qk; }
        else if (c < 2 * KD) { gch = key_dim + hk * KD + (c - KD); dst = &s_k[c - KD]; own = own_qk; }
        else { gch = 2 * key_dim + h * VD + col0 + (c - 2 * KD); dst = &s_v[c - 2 * KD]; own = true; }
        const float x = qkv[gch];
        const float4 rv = *reinterpret_cast<const float4 *>(ring + (size_t)gch * kConvRing);
        const float rr[kConvRing] = {rv.x, rv.y, rv.z, rv.w};
        const float *w = L.conv_w + (size_t)gch * K;
        float acc = 0.f;
        for (int j = 0; j < K - 1; j++) acc += w[j] * rr[ring_slot(ph, K, j)];
        acc += w[K - 1] * x;
        if (own) ring[(size_t)gch * kConvRing + (ph & (kConvRing - 1))] = x;
        *dst = omh_silu(acc);
    }
    if (tid == 0) {
        // gates (qwen.c:337-338)
        const float g = -expf(L.A_log[h]) * omh_softplus(args.a[tok * args.ld_ab + h] + L.dt_bias[h]);
        s_gam = expf(g);
        s_beta = omh_sigmoid(args.b[tok * args.ld_ab + h]);
        if (h == 0 && cs == 0) L.phase[(1 - L.epoch) * L.max_seqs + b] = (ph + 1) & (kConvRing - 1);
    }
    if (h == 0 && cs == 0 && b == 0) {
        // sequences outside this launch keep their phase in the other buffer
        for (int bb = args.B + tid; bb < L.max_seqs; bb += TPB)
            L.phase[(1 - L.epoch) * L.max_seqs + bb] = L.phase[L.epoch * L.max_seqs + bb];
    }
    omh_lds_barrier();
    // L2 norm of q and k (eps 1e-6), then q *= kd^-1/2 (qwen.c:153-157, 326-329)
    if (wave == 0) {
        float sq = 0.f, sk = 0.f;
        for (int i = lane; i < KD; i += OMH_WAVE) { sq += s_q[i] * s_q[i]; sk += s_k[i] * s_k[i]; }
        sq = omh_xor_sum_below<OMH_WAVE>(sq);
        sk = omh_xor_sum_below<OMH_WAVE>(sk);
        const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f);
        const float scale = 1.f / sqrtf((float)KD);
        for (int i = lane; i < KD; i += OMH_WAVE) { s_q[i] = (s_q[i] * rq) * scale; s_k[i] *= rk; }
    }
    omh_lds_barrier();

    // (3) delta rule on this slice of value head h (qwen.c:339-352)
    const float gam = s_gam, beta = s_beta;
    float4 kv = f4_zero();
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        s[m] = f4_scale(s[m], gam);
        kv = f4_fma(s[m], s_k[rg + RG * m], kv);
    }
    kv = colsum<C4, NW>(kv, s_red1, wave, lane, c4);
    const float4 vv = *reinterpret_cast<const float4 *>(&s_v[c4 * 4]);
    const float4 delta = f4_scale(f4_sub(vv, kv), beta);
    float4 o = f4_zero();
#pragma unroll
    for (int m = 0; m < RPT; m++) {
        const int i = rg + RG * m;
        s[m] = f4_fma(delta, s_k[i], s[m]);
        o = f4_fma(s[m], s_q[i], o);
        omh_st_stream(Sp + (size_t)i * VD + c4 * 4, s[m]);
    }
    o = colsum<C4, NW>(o, s_red2, wave, lane, c4);

    // (4) gated RMSNorm over the head's vd columns (qwen.c:353-357)
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = omh_xor_sum_below<C4>(ss);              // this slice's sum of squares
    float *core = args.core + tok * vdim + (size_t)h * VD;
    if constexpr (NCS == 1) {
        if (rg == 0) {
            const float rn = 1.f / sqrtf(ss / (float)VD + args.eps);
            *reinterpret_cast<float4 *>(core + c4 * 4) = gated(o, rn, gn, zz);
        }
    } else {
        // Cross-slice exchange with device-coherent (agent-scope) relaxed
        // atomics only: they bypass the per-XCD L2s, so no L2 write-back is
        // needed (an agent-scope fence would write back the whole L2).  Each
        // thread waits for its own stores to complete before the workgroup
        // barrier, and only then is the arrival counted.
        const size_t hb = (size_t)b * vh + h;
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
                const float rn = 1.f / sqrtf(tot / (float)VD + args.eps);
                const float *src = L.o_raw + hb * VD + tid * 4;
                float4 oo;
                oo.x = __hip_atomic_load(src + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oo.w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *reinterpret_cast<float4 *>(core + tid * 4) = gated(oo, rn, gn, zz);
            }
            if (tid == 0) __hip_atomic_store(L.cnt + hb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int KD, int VD, int NCS>
hipError_t launch_one(const DecodeArgs &a, hipStream_t st) {
    dim3 grid(a.vh * NCS, a.B, a.nl);
    hipLaunchKernelGGL((gdn_decode_core_kernel<KD, VD, NCS>), grid, dim3(DecShape<KD, VD, NCS>::TPB), 0, st, a);
    return hipGetLastError();
}

template <int KD, int VD>
hipError_t launch_ncs(const DecodeArgs &a, int ncs, hipStream_t st) {
    switch (ncs) {
        case 1: if constexpr (dec_valid<KD, VD, 1>()) return launch_one<KD, VD, 1>(a, st); break;
        case 2: if constexpr (dec_valid<KD, VD, 2>()) return launch_one<KD, VD, 2>(a, st); break;
        case 4: if constexpr (dec_valid<KD, VD, 4>()) return launch_one<KD, VD, 4>(a, st); break;
        case 8: if constexpr (dec_valid<KD, VD, 8>()) return launch_one<KD, VD, 8>(a, st); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

// One workgroup per value head is fastest on MI355X at every measured size:
// splitting columns multiplies the per-workgroup prologue and adds the
// exchange round trips, which cost more than the extra memory parallelism
// gains (30-layer B=1 step: 25.3 us at NCS=1 vs 36.1 us at NCS=4).
int default_ncs(int kd, int vd) {
    (void)kd; (void)vd;
    return 1;
}

}  // namespace

bool decode_core_supported(int kd, int vd, int rep, int K) {
    if (rep < 1 || K < 2 || K > kConvRing) return false;
    return (kd == vd && (kd == 16 || kd == 32 || kd == 64 || kd == 128)) || (kd == 32 && vd == 16);
}

hipError_t launch_decode_core(const DecodeArgs &a, int kd, int vd, int ncs, hipStream_t st) {
    if (!decode_core_supported(kd, vd, a.vh / a.kh, a.K)) return hipErrorInvalidValue;
    if (ncs <= 0) ncs = default_ncs(kd, vd);
    if (kd == 16 && vd == 16) return launch_ncs<16, 16>(a, ncs, st);
    if (kd == 32 && vd == 32) return launch_ncs<32, 32>(a, ncs, st);
    if (kd == 64 && vd == 64) return launch_ncs<64, 64>(a, ncs, st);
    if (kd == 128 && vd == 128) return launch_ncs<128, 128>(a, ncs, st);
    if (kd == 32 && vd == 16) return launch_ncs<32, 16>(a, ncs, st);
    return hipErrorInvalidValue;
}

}  // namespace omh
