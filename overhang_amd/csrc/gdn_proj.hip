// gdn_proj.hip — the layer's dense projections for few tokens (decode).
//
// y[t][o] = sum_i x[t][i] * W[o][i], with W either fp32 or int8 + per-row
// scale (the engine's QW twins, engines/qwen.c:34, 94-122, 124-138:
// dequantisation is acc * scale[o] after the fp32 dot product).  One
// wavefront owns one output row: it streams the row once from HBM (float4
// or 4 int8 per lane, fully coalesced) and applies it to the tokens in
// register tiles of 8, so the weights are read from HBM once per launch.
// The whole in_proj of a layer ([qkv | z] int8 + [b | a] fp32, or all fp32)
// is one launch: rows below n_q use the int8 matrix, the rest the fp32 one.
#include "omh_device.h"
#include "omh_internal.h"

namespace omh {
namespace {

constexpr int kProjWaves = 4;
constexpr int kProjTok = 8;

__global__ __launch_bounds__(kProjWaves * OMH_WAVE)
void proj_rows_kernel(const ProjArgs p) {
    const int lane = threadIdx.x % OMH_WAVE;
    const int o = blockIdx.x * kProjWaves + threadIdx.x / OMH_WAVE;
    if (o >= p.O) return;
    const bool q8 = o < p.n_q;
    const int8_t *qrow = q8 ? p.Q + (size_t)o * p.I : nullptr;
    const float *wrow = q8 ? nullptr : p.W + (size_t)(o - p.n_q) * p.I;
    const float sc = q8 ? p.scale[o] : 1.f;
    for (int t0 = 0; t0 < p.T; t0 += kProjTok) {
        const int nt = min(kProjTok, p.T - t0);
        float acc[kProjTok];
#pragma unroll
        for (int t = 0; t < kProjTok; t++) acc[t] = 0.f;
        for (int i = lane * 4; i < p.I; i += OMH_WAVE * 4) {
            float4 w;
            if (q8) {
                const char4 c = *reinterpret_cast<const char4 *>(qrow + i);
                w = make_float4((float)c.x, (float)c.y, (float)c.z, (float)c.w);
            } else {
                w = *reinterpret_cast<const float4 *>(wrow + i);
            }
#pragma unroll
            for (int t = 0; t < kProjTok; t++) {
                if (t < nt) {
                    const float4 xv = *reinterpret_cast<const float4 *>(p.x + (size_t)(t0 + t) * p.ldx + i);
                    acc[t] = fmaf(xv.x, w.x, acc[t]);
                    acc[t] = fmaf(xv.y, w.y, acc[t]);
                    acc[t] = fmaf(xv.z, w.z, acc[t]);
                    acc[t] = fmaf(xv.w, w.w, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kProjTok; t++) {
            const float v = omh_xor_sum_below<OMH_WAVE>(acc[t]);
            if (lane == 0 && t < nt) p.y[(size_t)(t0 + t) * p.ldy + o] = v * sc;
        }
    }
}

}  // namespace

hipError_t launch_proj(const ProjArgs &p, hipStream_t st) {
    if (p.O <= 0 || p.T <= 0) return hipSuccess;
    if (p.I % 4 != 0) return hipErrorInvalidValue;
    dim3 grid((p.O + kProjWaves - 1) / kProjWaves);
    hipLaunchKernelGGL(proj_rows_kernel, grid, dim3(kProjWaves * OMH_WAVE), 0, st, p);
    return hipGetLastError();
}

}  // namespace omh
