// attn.hip — the gated full-attention layer of the Qwen3.5/3.6 engine
// (engines/qwen.c:366-425, attn_step), the layer that every fourth block runs
// beside the GDN layers, for T new tokens of one sequence at positions
// pos .. pos+T-1.
//
// After the qkv projection (one launch_proj over the concatenated rows
// [H x (q | gate), KV x k, KV x v], qwen.c:370-374) three launches:
//  1. attn_prep_kernel, one wave per (token, head): RMSNorm of q and k with
//     (1 + w) weights (qwen.c:148-152, 385-386), partial RoPE over the first
//     rot dims as two non-interleaved halves (qwen.c:388-398, inverse
//     frequencies computed on the host as there), then q into a scratch row
//     and k, v into the sequence's cache rows pos + t (qwen.c:400-404).
//  2. attn_split_kernel, flash-decoding: one workgroup per (key split, kv
//     head, token) stages 64-key tiles of K and V through LDS once for all
//     the query heads of its group (GQA, qwen.c:408-409), keeps a running
//     max and sum per head (online softmax) and writes unnormalised
//     partials.  Lane = key for the scores (q broadcast from LDS), lane =
//     4 output columns for P.V (p broadcast from LDS).
//  3. attn_combine_kernel, one wave per (token, head): merges the splits,
//     normalises, and applies the output gate sigmoid(gate) (qwen.c:421).
// The o_proj is a second launch_proj.
//
// Decode is HBM-bound on the visible cache: 2 * KV * n * hd * 4 bytes for
// n = pos + 1 keys; the splits give >= 512 workgroups (two per CU).  Token t
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
    static constexpr int NW = 4;                  // waves
    static constexpr int GP = kAttnMaxGroup / NW; // query heads per wave, at most
    static constexpr size_t LDS = (size_t)(kAttnMaxGroup * HD + KT * KS + KT * HD + kAttnMaxGroup * KT) * sizeof(float);
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < OMH_WAVE; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, OMH_WAVE));
    return v;
}

template <int HD>
__global__ __launch_bounds__(OMH_WAVE) void attn_prep_kernel(const AttnArgs a) {
    constexpr int NE = (HD + OMH_WAVE - 1) / OMH_WAVE;
    __shared__ float sv[HD];
    const int H = a.H, KV = a.KV, nr = H + 2 * KV;
    const int t = blockIdx.x / nr, r = blockIdx.x % nr, lane = threadIdx.x;
    const int p = a.pos + t;
    const float *row = a.qkv + (size_t)t * a.ld_qkv;
    const float *src, *w = nullptr;
    float *dst;
    if (r < H) {                                   // q of head r (then its gate)
        src = row + (size_t)r * 2 * HD;
        w = a.qn;
        dst = a.qb + ((size_t)t * H + r) * HD;
    } else if (r < H + KV) {                       // k of kv head g
        const int g = r - H;
        src = row + (size_t)2 * H * HD + (size_t)g * HD;
        w = a.kn;
        dst = a.Kc + (((size_t)a.seq * KV + g) * a.max_t + p) * HD;
    } else {                                       // v of kv head g
        const int g = r - H - KV;
        src = row + (size_t)2 * H * HD + (size_t)(KV + g) * HD;
        dst = a.Vc + (((size_t)a.seq * KV + g) * a.max_t + p) * HD;
    }
    float v[NE];
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int j = lane + OMH_WAVE * i;
        v[i] = j < HD ? src[j] : 0.f;
    }
    if (w) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NE; i++) ss += v[i] * v[i];
        ss = omh_xor_sum_from<1>(ss);
        const float rr = 1.f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < HD) {
                v[i] = v[i] * rr * (1.f + w[j]);
                sv[j] = v[i];
            }
        }
        __syncthreads();
        const int half = a.rot / 2;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < a.rot) {
                const int jj = j < half ? j : j - half;
                const float ang = (float)p * a.inv[jj];
                const float cs = cosf(ang), sn = sinf(ang);
                const float a0 = sv[jj], b0 = sv[jj + half];
                v[i] = j < half ? a0 * cs - b0 * sn : b0 * cs + a0 * sn;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int j = lane + OMH_WAVE * i;
        if (j < HD) dst[j] = v[i];
    }
}

template <int HD>
__global__ __launch_bounds__(AttnShape<HD>::NW * OMH_WAVE) void attn_split_kernel(const AttnArgs a) {
    using S = AttnShape<HD>;
    constexpr int GP = S::GP, R4 = S::R4, NG4 = S::NG4, KT = S::KT, NT = S::NW * OMH_WAVE;
    extern __shared__ float smem[];
    float *qs = smem;                              // [group heads][HD]
    float *Ks = qs + kAttnMaxGroup * HD;           // [KT][KS]
    float *Vs = Ks + KT * S::KS;                   // [KT][HD]
    float *ps = Vs + KT * HD;                      // [group heads][KT]

    const int H = a.H, KV = a.KV, grp = H / KV, ns = a.ns;
    const int s = blockIdx.x % ns, g = (blockIdx.x / ns) % KV, t = blockIdx.x / (ns * KV);
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int n = a.pos + t + 1;                   // keys token t sees
    const int k0 = s * a.kps, k1 = min(n, k0 + a.kps);
    // partial of query head g*grp + i: index pb + i*ns
    const size_t pb = ((size_t)t * H + (size_t)g * grp) * ns + s;
    if (k0 >= k1) {                                // an empty split: weight zero in the merge
        if (tid < grp) {
            a.pml[2 * (pb + (size_t)tid * ns)] = -INFINITY;
            a.pml[2 * (pb + (size_t)tid * ns) + 1] = 0.f;
        }
        return;
    }
    for (int e = tid; e < grp * NG4; e += NT) {
        const int i = e / NG4, c = e % NG4;
        *reinterpret_cast<float4 *>(qs + i * HD + 4 * c) =
            *reinterpret_cast<const float4 *>(a.qb + ((size_t)t * H + (size_t)g * grp + i) * HD + 4 * c);
    }
    float m[GP], l[GP];
    float4 o[GP][R4];
#pragma unroll
    for (int i = 0; i < GP; i++) {
        m[i] = -INFINITY;
        l[i] = 0.f;
#pragma unroll
        for (int r = 0; r < R4; r++) o[i][r] = f4_zero();
    }
    const size_t cache0 = ((size_t)a.seq * KV + g) * a.max_t;
    const float *Kg = a.Kc + cache0 * HD, *Vg = a.Vc + cache0 * HD;

    for (int kt = k0; kt < k1; kt += KT) {
        const int nk = min(KT, k1 - kt);
        omh_lds_barrier();                         // the previous tile's readers are done
        for (int e = tid; e < nk * NG4; e += NT) {
            const int kk = e / NG4, c = e % NG4;
            const float4 kv = *reinterpret_cast<const float4 *>(Kg + (size_t)(kt + kk) * HD + 4 * c);
            const float4 vv = *reinterpret_cast<const float4 *>(Vg + (size_t)(kt + kk) * HD + 4 * c);
            *reinterpret_cast<float4 *>(Ks + kk * S::KS + 4 * c) = kv;
            *reinterpret_cast<float4 *>(Vs + kk * HD + 4 * c) = vv;
        }
        omh_lds_barrier();

        // scores q.k * hd^-1/2 (qwen.c:410-414), lane = key
        const bool valid = lane < nk;
        const float *kr = Ks + (valid ? lane : 0) * S::KS;
        float acc[GP];
#pragma unroll
        for (int i = 0; i < GP; i++) acc[i] = 0.f;
#pragma unroll 4
        for (int c = 0; c < NG4; c++) {
            const float4 kv = *reinterpret_cast<const float4 *>(kr + 4 * c);
#pragma unroll
            for (int i = 0; i < GP; i++) {
                const int h = wave + S::NW * i;
                if (h < grp) {
                    const float4 q = *reinterpret_cast<const float4 *>(qs + h * HD + 4 * c);
                    acc[i] = fmaf(q.x, kv.x, acc[i]);
                    acc[i] = fmaf(q.y, kv.y, acc[i]);
                    acc[i] = fmaf(q.z, kv.z, acc[i]);
                    acc[i] = fmaf(q.w, kv.w, acc[i]);
                }
            }
        }
        // online softmax (qwen.c:413 softmax_ over all keys, merged per tile)
#pragma unroll
        for (int i = 0; i < GP; i++) {
            const int h = wave + S::NW * i;
            if (h < grp) {
                const float sc = valid ? acc[i] * a.scale : -INFINITY;
                const float mn = fmaxf(m[i], wave_max(sc));
                const float corr = expf(m[i] - mn);
                const float pe = valid ? expf(sc - mn) : 0.f;
                l[i] = l[i] * corr + omh_xor_sum_from<1>(pe);
#pragma unroll
                for (int r = 0; r < R4; r++) o[i][r] = f4_scale(o[i][r], corr);
                ps[h * KT + lane] = pe;
                m[i] = mn;
            }
        }
        // ps rows are written and read by the same wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // P.V (qwen.c:415-419), lane = 4 columns
        for (int kk = 0; kk < nk; kk++) {
#pragma unroll
            for (int i = 0; i < GP; i++) {
                const int h = wave + S::NW * i;
                if (h < grp) {
                    const float pv = ps[h * KT + kk];
#pragma unroll
                    for (int r = 0; r < R4; r++) {
                        const int c = lane + OMH_WAVE * r;
                        if (c < NG4) o[i][r] = f4_fma(*reinterpret_cast<const float4 *>(Vs + kk * HD + 4 * c), pv, o[i][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < GP; i++) {
        const int h = wave + S::NW * i;
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

template <int HD>
__global__ __launch_bounds__(OMH_WAVE) void attn_combine_kernel(const AttnArgs a) {
    constexpr int NE = (HD + OMH_WAVE - 1) / OMH_WAVE;
    const int th = blockIdx.x, t = th / a.H, h = th % a.H, lane = threadIdx.x, ns = a.ns;
    const size_t pb = (size_t)th * ns;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, a.pml[2 * (pb + s)]);
    float L = 0.f, o[NE];
#pragma unroll
    for (int i = 0; i < NE; i++) o[i] = 0.f;
    for (int s = 0; s < ns; s++) {
        const float ms = a.pml[2 * (pb + s)];
        if (ms == -INFINITY) continue;             // empty split, partial never written
        const float wgt = expf(ms - M);
        L = fmaf(a.pml[2 * (pb + s) + 1], wgt, L);
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int j = lane + OMH_WAVE * i;
            if (j < HD) o[i] = fmaf(a.po[(pb + s) * HD + j], wgt, o[i]);
        }
    }
    const float rl = 1.f / L;                      // split 0 always holds key 0: L > 0
    const float *gate = a.qkv + (size_t)t * a.ld_qkv + (size_t)h * 2 * HD + HD;
    float *dst = a.ctx + ((size_t)t * a.H + h) * HD;
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int j = lane + OMH_WAVE * i;
        if (j < HD) dst[j] = o[i] * rl * omh_sigmoid(gate[j]);
    }
}

template <int HD>
hipError_t launch_attn_d(const AttnArgs &a, hipStream_t st) {
    static const bool lds_ok = hipFuncSetAttribute((const void *)attn_split_kernel<HD>,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)AttnShape<HD>::LDS) == hipSuccess;
    if (!lds_ok) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_prep_kernel<HD>), dim3((unsigned)(a.T * (a.H + 2 * a.KV))), dim3(OMH_WAVE), 0, st, a);
    hipLaunchKernelGGL((attn_split_kernel<HD>), dim3((unsigned)(a.ns * a.KV * a.T)),
                       dim3(AttnShape<HD>::NW * OMH_WAVE), AttnShape<HD>::LDS, st, a);
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3((unsigned)(a.T * a.H)), dim3(OMH_WAVE), 0, st, a);
    return hipGetLastError();
}

}  // namespace

bool attn_supported(int hd, int H, int KV, int rot) {
    return (hd == 32 || hd == 64 || hd == 128 || hd == 256) && KV >= 1 && H >= KV && H % KV == 0 &&
           H / KV <= kAttnMaxGroup && rot >= 0 && rot <= hd && rot % 2 == 0;
}

void attn_plan(int pos, int T, int KV, int &ns, int &kps) {
    const long nmax = (long)pos + T;                       // keys the last token sees
    const long per = (long)KV * T;
    const long want = per >= 512 ? 1 : (512 + per - 1) / per;   // splits for >= 512 workgroups
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
