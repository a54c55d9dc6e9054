// gdn_proj.hip — the layer's dense projections (in_proj and out_proj).
//
// y[t][o] = sum_i x[t][i] * W[o][i], with W either fp32 or int8 + per-row
// scale (the engine's QW twins, engines/qwen.c:34, 94-122, 124-138:
// dequantisation is acc * scale[o] after the fp32 dot product; the int8
// values are exact in fp32, so the products are the reference's).  The
// whole in_proj of a layer ([qkv | z] int8 + [b | a] fp32, or all fp32) is
// one launch: rows below n_q use the int8 matrix, the rest the fp32 one
// (n_q is a multiple of 16, so a 16-row tile is one or the other).
//
// Every kernel streams each weight row from HBM once per launch and token
// tile (the bound for decode batches), every lane reading 16 consecutive
// weights per load (16 B of int8 or 64 B of fp32):
//   * T <= 4 tokens: GEMV.  A wave takes 8 rows and one k-slice; lane l
//     covers k = 1024c + 16l + e of it, with the 8 rows' weights in flight
//     together; the 8 row sums are reduced over the lanes in one butterfly
//     and the k-slices through LDS.
//   * T > 4, int8 rows: exact bf16 x 3 products on the bf16 matrix cores
//     (proj_q8_wave_kernel: 64-row x 16 TT-token tiles per wave, operands
//     straight into registers; proj_q8_bf16x3_kernel for the shapes its
//     plan does not take), see the section further down.
//   * T > 4, fp32 rows: fp32 MFMA (16x16x4), tokens x rows tiles.  Within a
//     64-wide k block, lane (l%16, g) holds x and W at k = 16g + 4j + s for
//     its token / row l%16, so one 16-byte weight load and four float4 x
//     loads feed 16 MFMAs (the k order is permuted identically on both
//     operands).  A workgroup is RT row tiles x KS k-slices (RT * KS = 4
//     waves); the k-slices are summed through LDS.  Beside int8 rows the
//     fp32 rows run as extra workgroups of the int8 launch where they can.
#include "omh_device.h"
#include "omh_internal.h"
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace omh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

// s_waitcnt immediate for vmcnt(n) alone (expcnt and lgkmcnt not waited)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// s_waitcnt vmcnt(min(n, N)) for a wave-uniform n in 0..N (the count must be
// an immediate: a chain of compares)
template <int N>
__device__ __forceinline__ void wait_vmcnt(int n) {
    if (n >= N) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(N));
        return;
    }
    if constexpr (N > 0) wait_vmcnt<N - 1>(n);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>)
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// Weight fragment: 16 consecutive weights of one row, as loaded (int8 or
// fp32) and as fp32.
template <bool Q8>
struct WFrag;
template <>
struct WFrag<true> {
    int4 r;
    __device__ __forceinline__ void load(const ProjArgs &p, int row, int k) {
        r = *reinterpret_cast<const int4 *>(p.Q + (size_t)row * p.I + k);
    }
    // signed byte s = (u ^ 0x80) - 128 for its unsigned bits u: an
    // unsigned-byte conversion and an exact subtraction.  (A signed bitfield
    // extract followed by int->float is folded by this compiler into an SDWA
    // unsigned conversion of the sign-extended byte, which turns -1 into
    // 2^32 - 1.)
    __device__ __forceinline__ void unpack(float (&w)[16]) const {
        const unsigned v[4] = {(unsigned)r.x ^ 0x80808080u, (unsigned)r.y ^ 0x80808080u,
                               (unsigned)r.z ^ 0x80808080u, (unsigned)r.w ^ 0x80808080u};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int b = 0; b < 4; b++) w[4 * i + b] = (float)((v[i] >> (8 * b)) & 0xFFu) - 128.f;
    }
};
template <>
struct WFrag<false> {
    float4 f[4];
    __device__ __forceinline__ void load(const ProjArgs &p, int row, int k) {
        const float *src = p.W + (size_t)(row - p.n_q) * p.I + k;
#pragma unroll
        for (int i = 0; i < 4; i++) f[i] = *reinterpret_cast<const float4 *>(src + 4 * i);
    }
    __device__ __forceinline__ void unpack(float (&w)[16]) const {
#pragma unroll
        for (int i = 0; i < 4; i++) { w[4 * i] = f[i].x; w[4 * i + 1] = f[i].y; w[4 * i + 2] = f[i].z; w[4 * i + 3] = f[i].w; }
    }
};

__device__ __forceinline__ void load_x16(const float *src, float (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 f = *reinterpret_cast<const float4 *>(src + 4 * i);
        x[4 * i] = f.x; x[4 * i + 1] = f.y; x[4 * i + 2] = f.z; x[4 * i + 3] = f.w;
    }
}

// ---------------------------------------------------------------- GEMV
// Up to 4 tokens (decode).  int8 rows: a workgroup is 4 waves = RG row
// groups of kGemvRows rows x KS k-slices; a wave covers its k-slice in
// chunks of 1024 (16 per lane; one chunk per slice at the engine's shapes,
// where the slices are 1024 wide).  Per chunk the wave requests x first (an L2 hit after the launch's first
// waves), then every weight fragment of its rows, and sums the rows in
// that order: the load counter completes in issue order, so the
// conversion and products of the first rows run while the later rows'
// weights still stream in.  fp32 rows (in_proj's b/a rows, or a whole fp32
// matrix) take workgroups of their own, one row per wave over the full k,
// so their four-times wider weights do not leave a few workgroups
// straggling.  35B in_proj at one token with its weights from HBM (12288
// int8 rows + 64 fp32 rows, 25.7 MB), MI355X: 6.9 us, against 10.4 us with
// the fp32 rows inside the int8 workgroups and x requested after the
// weights (a plain read of the same bytes: 5.3 us).

// Rows per wave.  35B at one token, engine-order chain of 30 layers (in_proj
// 2048 -> 12352, out_proj 4096 -> 2048), MI355X: 18.2 us per layer with 4
// rows (in_proj 1536 workgroups, out_proj 512), 18.5 us with 8, 19.3 us
// with 2.
constexpr int kGemvRows = 4;
constexpr int kGemvCB = 1;            // chunks per request group

// Sum of v[i] over the 64 lanes for R (1, 2, 4 or 8) values at once,
// halving the set at each of the first log2 R exchanges (lane offsets 32,
// 16, 8), then summing the rest: lane L ends with the total of value
// gemv_row_of_lane<R>(L) (R = 8: 4*bit5(L) + 2*bit4(L) + bit3(L)).  The
// lane bits are tested once, up front: a test per select costs a compare
// and a hazard wait each.
template <int R>
__device__ __forceinline__ int gemv_row_of_lane(int lane) {
    const int b5 = (lane >> 5) & 1, b4 = (lane >> 4) & 1, b3 = (lane >> 3) & 1;
    return R == 8 ? 4 * b5 + 2 * b4 + b3 : (R == 4 ? 2 * b5 + b4 : (R == 2 ? b5 : 0));
}
// v of lane ^ OFF, on the VALU for OFF = 32 and 16 (permlane swaps; hi =
// the lane's bit OFF), 8 (row_ror:8), 2 and 1 (quad perms).  The swaps'
// results pass through an empty asm that keeps them in registers of their
// own (this compiler otherwise gave both the first one's register).
template <int OFF>
__device__ __forceinline__ float gemv_xor(float v, bool hi) {
    if constexpr (OFF == 32 || OFF == 16) {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        unsigned a, b;
        if constexpr (OFF == 32) {
            const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            a = p[0];
            b = p[1];
        } else {
            const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            a = p[0];
            b = p[1];
        }
        asm("" : "+v"(a), "+v"(b));
        return __builtin_bit_cast(float, hi ? a : b);
    } else if constexpr (OFF == 8) {
        return omh_dpp<0x128>(v);
    } else if constexpr (OFF == 2) {
        return omh_dpp<0x4E>(v);
    } else if constexpr (OFF == 1) {
        return omh_dpp<0xB1>(v);
    } else {
        return __shfl_xor(v, OFF, OMH_WAVE);
    }
}
// one halving exchange: lanes with hi keep the upper H values
template <int OFF, int H>
__device__ __forceinline__ void gemv_halve(float *c, bool hi) {
#pragma unroll
    for (int i = 0; i < H; i++) {
        const float send = hi ? c[i] : c[i + H];
        c[i] = (hi ? c[i + H] : c[i]) + gemv_xor<OFF>(send, hi);
    }
}
template <int R>
__device__ __forceinline__ float sum_rows_over_lanes(const float (&v)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per wave");
    const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8;
    float c[R];
#pragma unroll
    for (int i = 0; i < R; i++) c[i] = v[i];
    constexpr int LG = R == 8 ? 3 : (R == 4 ? 2 : (R == 2 ? 1 : 0));
    if constexpr (LG >= 1) gemv_halve<32, R / 2>(c, h5);
    if constexpr (LG >= 2) gemv_halve<16, R / 4>(c, h4);
    if constexpr (LG >= 3) gemv_halve<8, 1>(c, h3);
    // the rest of the butterfly (offsets 32 >> LG .. 1), each step adding
    // the partner's value in the same order as a plain xor butterfly
    float r = c[0];
    if constexpr (LG == 0) r += gemv_xor<32>(r, h5);
    if constexpr (LG <= 1) r += gemv_xor<16>(r, h4);
    if constexpr (LG <= 2) {
        r += gemv_xor<8>(r, h3);
        // lanes i and i ^ 8 now agree, so lane i - 4 (row_ror:4) holds the
        // value of lane i ^ 4
        r += omh_dpp<0x124>(r);
    } else {
        r += gemv_xor<4>(r, false);
    }
    r += gemv_xor<2>(r, false);
    r += gemv_xor<1>(r, false);
    return r;
}

// R int8 rows r0.. over k-slice ks of KS, NT tokens; the k-slices meet in
// LDS (red) and the first slice's wave stores (unless !store).  GN: x is a
// decode core's gated output before its 1 / rms, which is applied here as
// x is loaded (ProjArgs::gssq): the lane's 16 inputs lie in one head, whose
// slices' sums of squares (one 16-byte load) are requested with x, before
// the weights, and summed in slice order once the weights are requested.
template <int NT, int KS, int R, bool GN>
__device__ __forceinline__ void gemv_q8_rows(const ProjArgs &p, int r0, int ks, int lane,
                                             float (*red)[NT][OMH_WAVE], int rg, bool store) {
    float acc[R][NT];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[i][t] = 0.f;
    const int nrow = min(R, p.n_q - r0);
    const int klen = p.I / KS, kbeg = ks * klen, kend = kbeg + klen;
    for (int kc = kbeg; kc < kend; kc += kGemvCB * 16 * OMH_WAVE) {
        int kk[kGemvCB];
        bool live[kGemvCB];
#pragma unroll
        for (int c = 0; c < kGemvCB; c++) {
            const int k = kc + c * 16 * OMH_WAVE + 16 * lane;
            live[c] = k < kend;
            kk[c] = live[c] ? k : kend - 16;          // (in range; its products are skipped)
        }
        float x[kGemvCB][NT][16];
#pragma unroll
        for (int c = 0; c < kGemvCB; c++)
#pragma unroll
            for (int t = 0; t < NT; t++) load_x16(p.x + (size_t)t * p.ldx + kk[c], x[c][t]);
        constexpr int NC = GN ? kGemvCB : 1, NTG = GN ? NT : 1;
        float4 sq[NC][NTG];
        if constexpr (GN) {
            const int nh = p.I / p.gvd;
#pragma unroll
            for (int c = 0; c < kGemvCB; c++)
#pragma unroll
                for (int t = 0; t < NT; t++)
                    sq[c][t] = *reinterpret_cast<const float4 *>(p.gssq + ((size_t)t * nh + kk[c] / p.gvd) * 4);
        }
        __builtin_amdgcn_sched_barrier(0);            // x first, then the weights
        WFrag<true> wf[R][kGemvCB];
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int c = 0; c < kGemvCB; c++) wf[i][c].load(p, r0 + min(i, nrow - 1), kk[c]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (GN) {
            // the gated RMSNorm's 1 / rms (qwen.c:353-357), its sum in slice order
#pragma unroll
            for (int c = 0; c < kGemvCB; c++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    float ss = 0.f;
                    ss += sq[c][t].x;
                    ss += sq[c][t].y;
                    ss += sq[c][t].z;
                    ss += sq[c][t].w;
                    const float rn = rsqrtf(ss / (float)p.gvd + p.geps);
#pragma unroll
                    for (int e = 0; e < 16; e++) x[c][t][e] *= rn;
                }
        }
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int c = 0; c < kGemvCB; c++) {
                if (!live[c]) continue;
                float w[16];
                wf[i][c].unpack(w);
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][t] = fmaf(x[c][t][e], w[e], acc[i][t]);
            }
    }
    const int myrow = gemv_row_of_lane<R>(lane);
    float tot[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float v[R];
#pragma unroll
        for (int i = 0; i < R; i++) v[i] = acc[i][t];
        tot[t] = sum_rows_over_lanes<R>(v, lane);
    }
    if (KS > 1) {
        if (ks > 0)
#pragma unroll
            for (int t = 0; t < NT; t++) red[(ks - 1) * 4 + rg][t][lane] = tot[t];
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int j = 0; j < KS - 1; j++)
#pragma unroll
            for (int t = 0; t < NT; t++) tot[t] += red[j * 4 + rg][t][lane];
    }
    if (store && lane % (OMH_WAVE / R) == 0 && myrow < nrow) {
        const int o = r0 + myrow;
        const float sc = p.scale[o];
#pragma unroll
        for (int t = 0; t < NT; t++) p.y[(size_t)t * p.ldy + o] = tot[t] * sc;
    }
}

// One fp32 row over the full k, one wave, NT tokens: chunks of 256 (4 per
// lane), eight per request group, x first.
template <int NT>
__device__ __forceinline__ void gemv_f32_row(const ProjArgs &p, int row, int lane) {
    const float *W = p.W + (size_t)(row - p.n_q) * p.I;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.f;
    for (int kc = 0; kc < p.I; kc += 8 * 4 * OMH_WAVE) {
        int kk[8];
        bool live[8];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int k = kc + c * 4 * OMH_WAVE + 4 * lane;
            live[c] = k < p.I;
            kk[c] = live[c] ? k : p.I - 4;
        }
        float4 xv[NT][8], wv[8];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int c = 0; c < 8; c++) xv[t][c] = *reinterpret_cast<const float4 *>(p.x + (size_t)t * p.ldx + kk[c]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 8; c++) wv[c] = *reinterpret_cast<const float4 *>(W + kk[c]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if (!live[c]) continue;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                acc[t] = fmaf(xv[t][c].x, wv[c].x, acc[t]);
                acc[t] = fmaf(xv[t][c].y, wv[c].y, acc[t]);
                acc[t] = fmaf(xv[t][c].z, wv[c].z, acc[t]);
                acc[t] = fmaf(xv[t][c].w, wv[c].w, acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        // the xor butterfly over offsets 32 .. 1 on the VALU (gemv_xor)
        float a = acc[t];
        a += gemv_xor<32>(a, lane & 32);
        a += gemv_xor<16>(a, lane & 16);
        a += gemv_xor<8>(a, false);
        a += omh_dpp<0x124>(a);        // lane i - 4 holds lane i ^ 4's value once i and i ^ 8 agree
        a += gemv_xor<2>(a, false);
        a += gemv_xor<1>(a, false);
        if (lane == 0) p.y[(size_t)t * p.ldy + row] = a;
    }
}

// Workgroups 0 .. nwg8-1: the int8 rows; the rest: the fp32 rows, four per
// workgroup (one per wave).
template <int NT, int KS, int R, bool GN>
__global__ __launch_bounds__(4 * OMH_WAVE)
void proj_gemv_kernel(const ProjArgs p, int nwg8) {
    constexpr int RG = 4 / KS;
    __shared__ float red[KS > 1 ? (KS - 1) * 4 : 1][NT][OMH_WAVE];
    const int lane = threadIdx.x % OMH_WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / OMH_WAVE);
    if ((int)blockIdx.x >= nwg8) {
        const int row = p.n_q + ((int)blockIdx.x - nwg8) * 4 + wv;
        if (row < p.O) gemv_f32_row<NT>(p, row, lane);
        return;
    }
    const int rg = wv % RG, ks = wv / RG;
    // a row group past the int8 rows works on the last group instead (the
    // workgroup stays together for the k-slice reduction) and stores nothing
    const int rs = (blockIdx.x * RG + rg) * R;
    const int r0 = min(rs, ((p.n_q - 1) / R) * R);
    gemv_q8_rows<NT, KS, R, GN>(p, r0, ks, lane, red, rg, rs < p.n_q);
}

// ---------------------------------------------------------------- MFMA
constexpr int kMfmaTok = 64;            // tokens per workgroup (up to 4 tiles of 16)

// One wave: a 16-row tile x TT token tiles over k in [kbeg, kbeg + klen),
// nb = klen / 64 blocks, PF | nb.  The weights come in batches of PF blocks
// whose loads are all issued before the batch's x loads: the load counter
// completes in order, so waiting for an x fragment also waits for every
// weight load issued before it, and batching pays the HBM latency once per
// batch instead of once per step.  The x fragments (one per (block, token
// tile) step) are loaded XD steps ahead into NX = XD + 1 rotating 16-float
// buffers (L2 latency); the batch's step count PF * TT is a multiple of NX,
// so every buffer index is known at compile time.  Loads are unconditional
// (indices clamped at the end) so the wait counts are exact.
template <int TT, bool Q8, int PF>
__device__ __forceinline__ void mfma_tiles(const ProjArgs &p, int r0, int t0, int kbeg, int klen, int lane,
                                           v4f (&acc)[4]) {
    constexpr int NS = PF * TT;                          // steps per batch
    constexpr int NX = NS % 4 == 0 ? 4 : (NS % 2 == 0 ? 2 : 1);
    constexpr int XD = NX - 1 > 0 ? NX - 1 : 0;          // prefetch distance in steps
    const int l16 = lane % 16, g = lane / 16;
    const int row = min(r0 + l16, p.O - 1);
    const float *xr[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) xr[tt] = p.x + (size_t)min(t0 + 16 * tt + l16, p.T - 1) * p.ldx + 16 * g + kbeg;
    const int nb = klen / 64;
    const int kw = kbeg + 16 * g;
    // x of global step q (block q / TT, token tile q % TT), clamped to the last step
    auto load_step = [&](int q, float (&dst)[16]) {
        const int b = min(q / TT, nb - 1);
        load_x16(xr[q % TT] + 64 * b, dst);
    };
    float xs[NX][16];
    for (int b0 = 0; b0 < nb; b0 += PF) {
        WFrag<Q8> wq[PF];
#pragma unroll
        for (int i = 0; i < PF; i++) wq[i].load(p, row, kw + 64 * (b0 + i));
        if (b0 == 0)
#pragma unroll
            for (int q = 0; q < XD; q++) load_step(q, xs[q]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < PF; i++) {
            float w[16];
            wq[i].unpack(w);
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const int st = i * TT + tt;                     // step within the batch
                const int q = b0 * TT + st;                     // global step
                if (NX == 1) load_step(q, xs[0]);
                else load_step(q + XD, xs[(st + XD) % NX]);
                __builtin_amdgcn_sched_barrier(0);   // keep the prefetch ahead of the products
#pragma unroll
                for (int e = 0; e < 16; e++)
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[st % NX][e], w[e], acc[tt], 0, 0, 0);
            }
        }
    }
}

// One workgroup (bx, by) of the fp32-MFMA projection.
template <int RT, int TT, int PF>
__device__ __forceinline__ void proj_mfma_wg(const ProjArgs &p, int bx, int by) {
    constexpr int KS = 4 / RT;
    __shared__ v4f s_red[KS > 1 ? KS - 1 : 1][RT][TT][OMH_WAVE];
    const int lane = threadIdx.x % OMH_WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / OMH_WAVE);
    const int rt = wv % RT, ks = wv / RT;
    const int r0 = (bx * RT + rt) * 16;
    const int t0 = by * (TT * 16);
    const int klen = p.I / KS, kbeg = ks * klen;
    v4f acc[4];
#pragma unroll
    for (int tt = 0; tt < 4; tt++) acc[tt] = v4f{0.f, 0.f, 0.f, 0.f};
    if (r0 < p.O) {
        // (fp32 fragments are 4x the registers of int8 ones: batches of 2
        // blocks, except for a single 16 x 16 tile, whose 8 blocks fit)
        constexpr int PF32 = (RT == 1 && TT == 1) ? PF : (PF > 2 ? 2 : PF);
        if (r0 < p.n_q) mfma_tiles<TT, true, PF>(p, r0, t0, kbeg, klen, lane, acc);
        else mfma_tiles<TT, false, PF32>(p, r0, t0, kbeg, klen, lane, acc);
    }
    if (KS > 1) {
        if (ks > 0)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) s_red[ks - 1][rt][tt][lane] = acc[tt];
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int j = 0; j < KS - 1; j++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) acc[tt] += s_red[j][rt][tt][lane];
    }
    if (r0 >= p.O) return;
    const int l16 = lane % 16, g = lane / 16;
    const int o = r0 + l16;
    if (o >= p.O) return;
    const float sc = r0 < p.n_q ? p.scale[o] : 1.f;
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = t0 + 16 * tt + 4 * g + r;
            if (t < p.T) p.y[(size_t)t * p.ldy + o] = acc[tt][r] * sc;
        }
}

// XCD-aware order: the workgroup dispatched i-th runs on XCD i mod 8, and XCD
// x takes the x-th eighth of the (token block, row tile) pairs in row-major
// order, so the row tiles of a token block share an XCD and its L2 fetches
// the block's x once (dispatched in grid order, each XCD fetched it for every
// row tile; the 35B fp32 b / a rows at T = 4096: 26.2 -> 24.4 us).
template <int RT, int TT, int PF>
__global__ __launch_bounds__(4 * OMH_WAVE)
void proj_mfma_kernel(const ProjArgs p) {
    const unsigned nx = gridDim.x, n = nx * gridDim.y, i = blockIdx.x + nx * blockIdx.y;
    const unsigned m = n % 8 == 0 ? (i % 8) * (n / 8) + i / 8 : i;
    proj_mfma_wg<RT, TT, PF>(p, m % nx, m / nx);
}

template <int RT, int PF>
void launch_mfma_tt(const ProjArgs &p, dim3 grid, int tpw, hipStream_t st) {
    // token tiles per workgroup: all tiles when every workgroup sees one
    // token block, else tpw / 16 (the last block's missing tokens are clamped)
    const int tt = grid.y > 1 ? tpw / 16 : (p.T + 15) / 16;
    const dim3 blk(4 * OMH_WAVE);
    switch (tt) {
    case 1: hipLaunchKernelGGL((proj_mfma_kernel<RT, 1, PF>), grid, blk, 0, st, p); break;
    case 2: hipLaunchKernelGGL((proj_mfma_kernel<RT, 2, PF>), grid, blk, 0, st, p); break;
    case 3: hipLaunchKernelGGL((proj_mfma_kernel<RT, 3, PF>), grid, blk, 0, st, p); break;
    default: hipLaunchKernelGGL((proj_mfma_kernel<RT, 4, PF>), grid, blk, 0, st, p); break;
    }
}

template <int RT>
void launch_mfma_rt(const ProjArgs &p, dim3 grid, int tpw, hipStream_t st) {
    const int nb = p.I / (4 / RT) / 64;       // 64-wide blocks per k-slice
    if (nb % 8 == 0) launch_mfma_tt<RT, 8>(p, grid, tpw, st);
    else if (nb % 2 == 0) launch_mfma_tt<RT, 2>(p, grid, tpw, st);
    else launch_mfma_tt<RT, 1>(p, grid, tpw, st);
}

// ---------------------------------------------------------------- int8 rows, T > 4: bf16 x 3
// int8 weights are exact in bf16, and x splits exactly into three bf16
// terms, x = hi + mid + lo (hi = bf16(x), mid = bf16(x - hi), lo = the
// rest, which has at most 8 significant bits left), so
// sum_i x_i w_i = sum_i (hi_i w_i + mid_i w_i + lo_i w_i) with every product
// exact, accumulated in fp32 on the bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16).  x is split once per launch into three bf16
// planes [3][T][I] (proj_split_x_kernel); a workgroup of RG row groups x KS
// k-slices of waves (RG * KS = 4) stages, per 64-wide k block, the planes'
// rows of its 16 * TT tokens in LDS (double-buffered, shared by the RG waves
// of a k-slice), while each wave streams its weights (16 B of int8 per lane
// per row tile and block) PF blocks ahead.  A wave owns RW = 2 tiles of 16
// rows.  Operand layout of a 32-wide k step s: lane (l%16, g) holds rows /
// tokens l%16 at k = 16g + 8s + j, j < 8 (the same permutation of k on both
// operands).
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr int kQ8Rows = 32;                 // rows per wave
constexpr int kQ8K = 64;                    // k per staged block
constexpr int kQ8Tok = 32;                  // tokens per workgroup

// planes[p] = term p of x in the chunk layout (xpiece), and the sum of x[t][k]
// over each 64-wide k block (sums[t][k / 64], after the planes); 8 values
// per thread
// (block 0 also clears the k-split arrival counters of the launch after it)
__global__ __launch_bounds__(256)
void proj_split_x_kernel(const float *__restrict__ x, int64_t ldx, uint16_t *__restrict__ xb, int T, int I, int *cnt,
                         int ncnt) {
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < ncnt; i += 256) cnt[i] = 0;
    const size_t n8 = (size_t)T * (I / 8);
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = e < n8;
    const size_t ec = live ? e : n8 - 1;
    const int t = (int)(ec / (I / 8)), k = (int)(ec % (I / 8)) * 8;
    const float4 a = *reinterpret_cast<const float4 *>(x + (size_t)t * ldx + k);
    const float4 b = *reinterpret_cast<const float4 *>(x + (size_t)t * ldx + k + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    v8bf hi, mid, lo;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        hi[j] = (__bf16)v[j];
        const float r1 = v[j] - (float)hi[j];
        mid[j] = (__bf16)r1;
        lo[j] = (__bf16)(r1 - (float)mid[j]);
        sum += v[j];
    }
    // the 8 threads of a 64-wide block are 8 consecutive lanes (I % 64 == 0)
    sum += __shfl_xor(sum, 1, OMH_WAVE);
    sum += __shfl_xor(sum, 2, OMH_WAVE);
    sum += __shfl_xor(sum, 4, OMH_WAVE);
    if (!live) return;
    const size_t plane = (size_t)T * I, o = xpiece(k / 8, t, T, I);
    *reinterpret_cast<v8bf *>(xb + o) = hi;
    *reinterpret_cast<v8bf *>(xb + plane + o) = mid;
    *reinterpret_cast<v8bf *>(xb + 2 * plane + o) = lo;
    if (k % 64 == 0) reinterpret_cast<float *>(xb + 3 * plane)[(size_t)t * (I / 64) + k / 64] = sum;
}

// 8 int8 weights w as bf16 of u = w + 128 (0..255, exact in bf16): one
// unsigned-byte conversion per value and one pack per pair; the products
// then carry + 128 x, which the epilogue takes off as 128 * (sum of x)
__device__ __forceinline__ v8bf q8_to_bf16_u(unsigned lo, unsigned hi) {
    const unsigned u[2] = {lo ^ 0x80808080u, hi ^ 0x80808080u};
    v8bf r;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int b = 0; b < 4; b++) r[4 * i + b] = (__bf16)(float)((u[i] >> (8 * b)) & 0xFFu);
    return r;
}

// NBC: the k blocks per slice when known at compile time (the loop is then
// straight-line: across a loop back edge the compiler's load-counter waits
// fall back to draining the prefetched blocks), else 0
template <int RG, int KS, int TT, int PF, int NBC>
__global__ __launch_bounds__(4 * OMH_WAVE)
void proj_q8_bf16x3_kernel(const ProjArgs p) {
    constexpr int RW = kQ8Rows / 16, KB = kQ8K, XR = KB + 8;     // padded staging row (bf16)
    constexpr int NST = KB / 32;                                 // 32-wide MFMA steps per block
    constexpr int NW4 = KB / 64;                                 // 16-byte weight loads per row tile and block
    constexpr int NU4 = KS * 3 * TT * 16 * (KB / 8) / (4 * OMH_WAVE);   // 16-byte x pieces per thread per block
    static_assert(NU4 >= 1 && KS * 3 * TT * 16 * (KB / 8) % (4 * OMH_WAVE) == 0, "x staging split");
    __shared__ __align__(16) __bf16 xs[2][KS][3][TT * 16][XR];
    __shared__ v4f s_red[KS > 1 ? KS - 1 : 1][RG][RW][TT][OMH_WAVE];

    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int rg = wv % RG, ks = wv / RG;
    const int l16 = lane % 16, g = lane / 16;
    const int r0 = (blockIdx.x * RG + rg) * kQ8Rows;
    const int t0 = blockIdx.y * (TT * 16);
    const int klen = p.I / KS, nb = NBC > 0 ? NBC : klen / KB;
    const size_t plane = (size_t)p.T * p.I;

    // x staging: piece f of block b -> (k-slice, term, token, 16-byte column),
    // XD blocks ahead in a ring of registers
    constexpr int XD0 = NU4 <= 3 ? 4 : (NU4 <= 6 ? 2 : 1);
    constexpr int XD = XD0 < PF ? XD0 : PF;
    static_assert(PF % XD == 0, "ring slots known at compile time");
    v4u xr[XD][NU4];       // (a clang vector: the HIP uint4 struct is copied through memory)
    auto piece = [&](int f, int &kq, int &sp, int &t, int &c) __attribute__((always_inline)) {
        const int idx = tid + f * 4 * OMH_WAVE;
        c = idx % (KB / 8);
        t = (idx / (KB / 8)) % (TT * 16);
        sp = (idx / (KB / 8 * TT * 16)) % 3;
        kq = idx / (KB / 8 * TT * 16 * 3);
    };
    // (slot is a compile-time constant at every call, so the ring stays in
    // registers)
    auto x_load = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
        b = min(b, nb - 1);
#pragma unroll
        for (int f = 0; f < NU4; f++) {
            int kq, sp, t, c;
            piece(f, kq, sp, t, c);
            xr[slot][f] = *reinterpret_cast<const v4u *>(
                p.xb + sp * plane + xpiece((kq * klen + b * KB) / 8 + c, min(t0 + t, p.T - 1), p.T, p.I));
        }
    };
    auto x_stage = [&](int buf, auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
#pragma unroll
        for (int f = 0; f < NU4; f++) {
            int kq, sp, t, c;
            piece(f, kq, sp, t, c);
            *reinterpret_cast<v4u *>(&xs[buf][kq][sp][t][8 * c]) = xr[slot][f];
        }
    };

    // weights: KB / 4 int8 per lane per row tile and block, PF blocks ahead;
    // lane group g holds k = (KB / 4) g + 8 s + j of step s
    const int8_t *wrow[RW];
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
        wrow[rw] = p.Q + (size_t)min(r0 + 16 * rw + l16, p.O - 1) * p.I + ks * klen + (KB / 4) * g;
    int4 wq[PF][RW][NW4];
    auto w_load = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int slot = decltype(slot_c)::value;
#pragma unroll
        for (int rw = 0; rw < RW; rw++)
#pragma unroll
            for (int h = 0; h < NW4; h++)
                wq[slot][rw][h] = *reinterpret_cast<const int4 *>(wrow[rw] + (size_t)min(b, nb - 1) * KB + 16 * h);
    };

    v4f acc[RW][TT];
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[rw][tt] = v4f{0.f, 0.f, 0.f, 0.f};

    // the prologue issues x then w per block, as the loop does, so the wait
    // counts are the same on entry and on the back edge
    static_for<PF>([&](auto sc) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        if constexpr (s < XD) x_load(s, std::integral_constant<int, s>{});
        w_load(s, sc);
    });
    x_stage(0, std::integral_constant<int, 0>{});
    x_load(XD, std::integral_constant<int, 0>{});
    // PF divides nb
    auto step = [&](int b0) __attribute__((always_inline)) {
        static_for<PF>([&](auto sc) __attribute__((always_inline)) {
            constexpr int s = decltype(sc)::value;
            const int b = b0 + s;
            const int buf = b & 1;
            // no code motion across blocks: the weights of a block are
            // unpacked only after its loads (PF blocks old) are in
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();                     // block b staged; every wave is past block b-1
            // every x operand of the block read at once (one LDS latency);
            // block b+1 staged into the other buffer while this block's
            // products run (its writes are done by the next barrier); the
            // weights unpacked meanwhile, then the products
            v4u B[NST][TT][3];
            v8bf A[NST][RW];
#pragma unroll
            for (int st = 0; st < NST; st++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int sp = 0; sp < 3; sp++)
                        B[st][tt][sp] = *reinterpret_cast<const v4u *>(&xs[buf][ks][sp][16 * tt + l16][(KB / 4) * g + 8 * st]);
            x_stage(buf ^ 1, std::integral_constant<int, (s + 1) % XD>{});
            x_load(b + 1 + XD, std::integral_constant<int, (s + 1) % XD>{});
#pragma unroll
            for (int rw = 0; rw < RW; rw++)
#pragma unroll
                for (int st = 0; st < NST; st++) {
                    const int4 w = wq[s][rw][st / 2];
                    A[st][rw] = st % 2 == 0 ? q8_to_bf16_u((unsigned)w.x, (unsigned)w.y) : q8_to_bf16_u((unsigned)w.z, (unsigned)w.w);
                }
#pragma unroll
            for (int st = 0; st < NST; st++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int sp = 0; sp < 3; sp++)
#pragma unroll
                        for (int rw = 0; rw < RW; rw++)
                            acc[rw][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[st][rw], __builtin_bit_cast(v8bf, B[st][tt][sp]),
                                                                                  acc[rw][tt], 0, 0, 0);
            w_load(b + PF, sc);
        });
    };
    if constexpr (NBC > 0) {
#pragma unroll
        for (int b0 = 0; b0 < NBC; b0 += PF) step(b0);
    } else {
        for (int b0 = 0; b0 < nb; b0 += PF) step(b0);
    }

    // sum x (w + 128) - 128 sum x = sum x w, the sums of the k-slice's
    // 64-wide blocks from the split kernel
    {
        const float *sums = reinterpret_cast<const float *>(p.xb + 3 * plane);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const float *sr = sums + (size_t)min(t0 + 16 * tt + l16, p.T - 1) * (p.I / 64) + ks * (klen / 64);
            // (independent loads in flight, not one L2 round trip per block)
            float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const int nq = klen / 64;
            int q = 0;
            for (; q + 8 <= nq; q += 8)
#pragma unroll
                for (int u = 0; u < 8; u++) part[u] += sr[q + u];
            for (; q < nq; q++) part[0] += sr[q];
            const float sx = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
#pragma unroll
            for (int rw = 0; rw < RW; rw++) acc[rw][tt] -= 128.f * sx;
        }
    }
    if (KS > 1) {
        if (ks > 0)
#pragma unroll
            for (int rw = 0; rw < RW; rw++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++) s_red[ks - 1][rg][rw][tt][lane] = acc[rw][tt];
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int j = 0; j < KS - 1; j++)
#pragma unroll
            for (int rw = 0; rw < RW; rw++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++) acc[rw][tt] += s_red[j][rg][rw][tt][lane];
    }
    // lane holds rows 4g .. 4g+3 of row tile rw for token l16 of token tile tt
#pragma unroll
    for (int rw = 0; rw < RW; rw++) {
        const int o = r0 + 16 * rw + 4 * g;
        if (o >= p.O) continue;
        const float4 sc = *reinterpret_cast<const float4 *>(p.scale + o);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const int t = t0 + 16 * tt + l16;
            if (t >= p.T) continue;
            float4 y;
            y.x = acc[rw][tt][0] * sc.x;
            y.y = acc[rw][tt][1] * sc.y;
            y.z = acc[rw][tt][2] * sc.z;
            y.w = acc[rw][tt][3] * sc.w;
            *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) = y;
        }
    }
}

// ------------------------------------------------ int8 rows, wave tiles
// The int8 rows on the bf16 matrix cores with a 64-row x 64-token output
// tile per wave: each x fragment (16 tokens x one 32-wide k step of one
// bf16 plane) feeds 4 row tiles and each weight fragment 4 token tiles x 3
// planes.  A wave then needs 256 B of x and 43 B of weights per 16x16x32
// product, loaded straight into registers (the x planes stay in L2, the
// weights stream from HBM three blocks ahead), so no operand goes through
// LDS and the main loop has no barriers.  The 4 waves of a workgroup take
// consecutive k-subslices of the same tile and are summed through LDS in
// wave order.  With few rows, G workgroups split k further: each stores
// its partial tile, and the last of the G to arrive (arrival counter) sums
// the G tiles in order, so the result does not depend on arrival order
// (device-coherent atomic stores and loads, as the sliced decode norm).
// Operand k order within a 128-wide superblock (the x plane layout,
// xpiece): lane (l%16, g) holds k = 32g + 8s + j of step s < 4, j < 8, on
// both operands; a weight "block" of the rings below is half a superblock
// (16 bytes per lane: steps 0-1 or 2-3).
constexpr int kWvRows = 64, kWvK = 64;

// Rows beside the int8 ones in the same launch: the fp32 rows of the
// projection (the b / a rows of in_proj), run by kF32Wgs extra workgroups
// of the fp32-MFMA path (one 16-row tile x 16 tokens each, k split over
// its 4 waves), appended along x after the int8 row groups, so they run
// alongside the int8 tiles instead of in a launch of their own.
struct F32Part {
    ProjArgs p;    // the fp32 rows as a projection of their own (n_q = 0)
    int nrg;       // int8 row groups (gridDim.x without the extra workgroups)
    int gx, nwg;   // fp32 workgroup grid width and count
};

template <int G, int WD, bool F32, int TT>
__global__ __launch_bounds__(4 * OMH_WAVE, 1)
void proj_q8_wave_kernel(const ProjArgs p, int nb, const F32Part f) {
    constexpr int RW = kWvRows / 16, NTOK = 16 * TT;          // rows and tokens of a wave's tile
    constexpr int kTileFloats = kWvRows * NTOK;               // one partial tile
    if constexpr (F32) {
        if ((int)blockIdx.x >= f.nrg) {
            const int i = (blockIdx.x - f.nrg) + (gridDim.x - f.nrg) * blockIdx.y;
            if (i < f.nwg) proj_mfma_wg<1, 1, 8>(f.p, i % f.gx, i / f.gx);
            return;
        }
    }
    __shared__ v4f s_red[4][RW][TT][OMH_WAVE];
    __shared__ float s_sx[NTOK];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, gq = lane / 16;
    const int r0 = blockIdx.x * kWvRows, t0 = blockIdx.y * NTOK;
    const int g = blockIdx.z;
    const int k0 = (g * 4 + w) * (nb * kWvK);
    const size_t plane = (size_t)p.T * p.I;

    // sum of x per token for the epilogue, from the split kernel's sums of
    // 64-wide blocks: TPT consecutive threads share a token, each taking
    // 1 / TPT of its blocks.  Requested first, summed after the main loop
    // (one load latency for the whole launch, hidden under it).
    constexpr int kSxRegs = 16, TPT = 4 * OMH_WAVE / NTOK;
    const int nq = p.I / 64, nqt = nq / TPT;
    const float *sq = reinterpret_cast<const float *>(p.xb + 3 * plane) + (size_t)min(t0 + tid / TPT, p.T - 1) * nq +
                      (tid % TPT) * nqt;
    float sxr[kSxRegs];
#pragma unroll
    for (int j = 0; j < kSxRegs; j++) sxr[j] = sq[min(j, nqt - 1)];

    const int8_t *wp[RW];
    const uint16_t *xp[TT];
#pragma unroll
    for (int rw = 0; rw < RW; rw++) wp[rw] = p.Q + (size_t)min(r0 + 16 * rw + l16, p.O - 1) * p.I + k0 + 32 * gq;
#pragma unroll
    for (int tt = 0; tt < TT; tt++) xp[tt] = p.xb + (size_t)min(t0 + 16 * tt + l16, p.T - 1) * 32 + 8 * gq;
    const size_t chunk = (size_t)p.T * 32;        // one 32-value chunk of every token

    // x XD - 1 steps ahead (two 32-wide steps per block) in a ring of XD
    // register slots, the weights WD blocks ahead in a ring of WD.  The loop
    // body is WD blocks, one period of both rings (XD divides 2 WD), so
    // every slot index is a compile-time constant; the loop stays a loop (a
    // fully unrolled body outruns the instruction cache: every wave would
    // run thousands of instructions exactly once).  Order within the loop:
    // at the start of step q the x of step q + XD - 1, after block b the
    // weights of block b + WD.  The prologue issues the loads of the
    // iteration before the first, in that order (those of negative steps
    // and blocks left out), so the wait counts agree on both edges into
    // the loop.
    constexpr int XD = 2;
    static_assert((2 * WD) % XD == 0, "ring periods");
    int4 wq[WD][RW];
    v4u xq[XD][TT][3];
    auto w_load = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
        b = min(b, nb - 1);
#pragma unroll
        for (int rw = 0; rw < RW; rw++)
            wq[sl][rw] = *reinterpret_cast<const int4 *>(wp[rw] + (b / 2) * (2 * kWvK) + 16 * (b % 2));
    };
    auto x_load = [&](int q, auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
        q = min(q, 2 * nb - 1);
        const size_t off = (size_t)(2 * (k0 / kWvK) + q) * chunk;   // step q of the wave's k range
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int sp = 0; sp < 3; sp++) xq[sl][tt][sp] = *reinterpret_cast<const v4u *>(xp[tt] + sp * plane + off);
    };

    v4f acc[RW][TT];
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[rw][tt] = v4f{0.f, 0.f, 0.f, 0.f};

    // step st of a block from x slot xs and weight slot ws
    auto step = [&](auto xs_c, auto ws_c, auto st_c) __attribute__((always_inline)) {
        constexpr int xs = decltype(xs_c)::value, ws = decltype(ws_c)::value, st = decltype(st_c)::value;
        v8bf A[RW];
#pragma unroll
        for (int rw = 0; rw < RW; rw++) {
            const int4 w4 = wq[ws][rw];
            A[rw] = st == 0 ? q8_to_bf16_u((unsigned)w4.x, (unsigned)w4.y) : q8_to_bf16_u((unsigned)w4.z, (unsigned)w4.w);
        }
#pragma unroll
        for (int sp = 0; sp < 3; sp++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int rw = 0; rw < RW; rw++)
                    acc[rw][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        A[rw], __builtin_bit_cast(v8bf, xq[xs][tt][sp]), acc[rw][tt], 0, 0, 0);
    };
    // the loads of one loop iteration's step u (0 <= u < 2 WD) relative to
    // its first block b0, with step u's products in between when run
    auto loads_at = [&](int b0, auto uc, auto run) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        const int q = 2 * b0 + u;
        __builtin_amdgcn_sched_barrier(0);
        if (q + XD - 1 >= 0) x_load(q + XD - 1, std::integral_constant<int, (u + XD - 1) % XD>{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(run)::value)
            step(std::integral_constant<int, u % XD>{}, std::integral_constant<int, u / 2>{}, std::integral_constant<int, u % 2>{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (u % 2 == 1)
            if (b0 + u / 2 + WD >= 0) w_load(b0 + u / 2 + WD, std::integral_constant<int, u / 2>{});
    };
    // prologue: the previous iteration's loads (b0 = -WD), without products
    static_for<2 * WD>([&](auto uc) __attribute__((always_inline)) { loads_at(-WD, uc, std::false_type{}); });
#pragma unroll 1
    for (int b0 = 0; b0 < nb; b0 += WD) {
        // (the scheduler would otherwise sink each prefetch next to its
        // use, where its wait drains everything in flight)
        static_for<2 * WD>([&](auto uc) __attribute__((always_inline)) { loads_at(b0, uc, std::true_type{}); });
    }

    // the workgroup's 4 k-subslices, in wave order; wave w then finishes
    // row tile w
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) s_red[w][rw][tt][lane] = acc[rw][tt];
    {
        float sx = 0.f;
#pragma unroll
        for (int j = 0; j < kSxRegs; j++) sx += j < nqt ? sxr[j] : 0.f;
        for (int j = kSxRegs; j < nqt; j++) sx += sq[j];
#pragma unroll
        for (int off = 1; off < TPT; off <<= 1) sx += __shfl_xor(sx, off, OMH_WAVE);
        if (tid % TPT == 0) s_sx[tid / TPT] = sx;
    }
    __syncthreads();
    v4f y[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
        y[tt] = ((s_red[0][w][tt][lane] + s_red[1][w][tt][lane]) + s_red[2][w][tt][lane]) + s_red[3][w][tt][lane];

    if constexpr (G > 1) {
        const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
        float *mine = p.part + (tile * G + g) * kTileFloats;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            float *d = mine + ((w * TT + tt) * OMH_WAVE + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; r++) __hip_atomic_store(d + r, y[tt][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);           // this thread's stores are complete
        __syncthreads();
        if (tid == 0) s_last = __hip_atomic_fetch_add(p.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
        __syncthreads();
        if (!s_last) return;
        // all G partial tiles requested at once, then summed in order
        v4f pt[G][TT];
#pragma unroll
        for (int gg = 0; gg < G; gg++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const float *q = p.part + (tile * G + gg) * kTileFloats + ((w * TT + tt) * OMH_WAVE + lane) * 4;
#pragma unroll
                for (int r = 0; r < 4; r++) pt[gg][tt][r] = __hip_atomic_load(q + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            y[tt] = pt[0][tt];
#pragma unroll
            for (int gg = 1; gg < G; gg++) y[tt] += pt[gg][tt];
        }
        if (tid == 0) __hip_atomic_store(p.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // sum x (w + 128) - 128 sum x = sum x w, times the row scales
#pragma unroll
    for (int tt = 0; tt < TT; tt++) y[tt] -= 128.f * s_sx[16 * tt + l16];
    // lane holds rows 4g .. 4g+3 of row tile w for token l16 of token tile tt
    const int o = r0 + 16 * w + 4 * gq;
    if (o >= p.O) return;
    const float4 sc = *reinterpret_cast<const float4 *>(p.scale + o);
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int t = t0 + 16 * tt + l16;
        if (t >= p.T) continue;
        float4 v;
        v.x = y[tt][0] * sc.x;
        v.y = y[tt][1] * sc.y;
        v.z = y[tt][2] * sc.z;
        v.w = y[tt][3] * sc.w;
        *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) = v;
    }
}

// ------------------------------------------- int8 rows, int8 matrix cores
// x as three int8 planes with a power-of-two scale per (token, 128-wide k
// block) (i8_off layout, omh_i8_split), so every product is int8 x int8 on
// v_mfma_i32_16x16x64_i8 and exact in int32: per block and plane a wave
// sums q * p over the block's 128 k exactly, then combines the three planes
// and the block scale in fp32, y += 2^E (A1 + (128 A2 + A3) 2^-14), and the
// row scale multiplies at the end (qwen.c:116-121).  The one approximation is
// x's representation, |x - x^| <= 2^-20 max|x| per block.  The weights go
// into the matrix cores as they are stored: no conversion.
//
// A wave owns a 64-row x 16 TT-token output tile; each weight fragment
// (16 rows x 64 k, 16 bytes per lane) feeds TT x 3 products, each x fragment
// 4.  The 4 waves of a workgroup take consecutive k-subslices of the tile
// and are summed through LDS in wave order; with few rows G workgroups split
// k further (partial tiles + arrival counter, summed in order by the last).
// Operands go straight from L2 / HBM into registers, one block ahead.  Tiles
// are numbered token tile fastest and dealt out so that one XCD runs the
// token tiles of a row group back to back: workgroups go to the XCDs in turn
// (workgroup i to XCD i mod 8), so tile (i mod 8) * per + i / 8 keeps a row
// group's weights in one L2.
typedef int v4i __attribute__((ext_vector_type(4)));

// x -> int8 planes with one scale per token (the power of two of the row's
// max|x|, written into every block's scale entry): one workgroup per token
// row, a float4 per thread per 1024 columns, read once (up to I = 4096 the
// row stays in registers between the max and the split).  Workgroup 0 also
// clears the k-split arrival counters.
__global__ __launch_bounds__(256)
void proj_split_i8_kernel(const float *__restrict__ x, int64_t ldx, int8_t *__restrict__ xb, int T, int I, int *cnt,
                          int ncnt) {
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < ncnt; i += 256) cnt[i] = 0;
    const int t = blockIdx.x;
    if (t >= T) return;
    constexpr int kRegs = 4;                                // float4s per thread kept in registers (I <= 4096)
    __shared__ float s_m[4];
    const float *xr = x + (size_t)t * ldx;
    float4 v[kRegs];
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < kRegs; j++) {
        const int k = 4 * threadIdx.x + 1024 * j;
        v[j] = k < I ? *reinterpret_cast<const float4 *>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    for (int k = 4 * threadIdx.x + 1024 * kRegs; k < I; k += 1024) {
        const float4 u = *reinterpret_cast<const float4 *>(xr + k);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
    }
    m = omh_lane_max(m);
    if (threadIdx.x % OMH_WAVE == 0) s_m[threadIdx.x / OMH_WAVE] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    const int E = omh_i8_exponent(m);
    const size_t plane = i8_plane_bytes(T, I);
    auto put = [&](int k, float4 u) __attribute__((always_inline)) {
        char4 a, b, c;
        int8_t t1, t2, t3;
        omh_i8_split(u.x, E, t1, t2, t3); a.x = t1; b.x = t2; c.x = t3;
        omh_i8_split(u.y, E, t1, t2, t3); a.y = t1; b.y = t2; c.y = t3;
        omh_i8_split(u.z, E, t1, t2, t3); a.z = t1; b.z = t2; c.z = t3;
        omh_i8_split(u.w, E, t1, t2, t3); a.w = t1; b.w = t2; c.w = t3;
        const size_t o = i8_off(k, t, T);
        *reinterpret_cast<char4 *>(xb + o) = a;
        *reinterpret_cast<char4 *>(xb + plane + o) = b;
        *reinterpret_cast<char4 *>(xb + 2 * plane + o) = c;
    };
#pragma unroll
    for (int j = 0; j < kRegs; j++) {
        const int k = 4 * threadIdx.x + 1024 * j;
        if (k < I) put(k, v[j]);
    }
    for (int k = 4 * threadIdx.x + 1024 * kRegs; k < I; k += 1024) put(k, *reinterpret_cast<const float4 *>(xr + k));
    const float sc = ldexpf(1.f, E);
    for (int kb = threadIdx.x; kb < I / kI8Blk; kb += 256) reinterpret_cast<float *>(xb + kI8Planes * plane)[(size_t)kb * T + t] = sc;
}

// The same split for many tokens: one workgroup of 16 waves per 16-token
// tile.  First each token's max |x| (wave w reads token w, a float4 per lane
// per 256 columns, eight loads in flight); then every 1 KiB fragment of the
// tile (one 64-wide k half-block, in i8_off order) is written whole by one
// wave, lane (l16, g) splitting token l16's x at k = 64 j + 16 g .. +15 (the
// row again, now from L2) into three 16-byte stores, so every store
// instruction writes one contiguous 1 KiB run per plane.  (With 4 waves per
// workgroup, one workgroup per CU, the loads' latency set the time: 29.7 us
// for 4096 tokens of 2048.)
constexpr int kSplitTileWaves = 16;
__global__ __launch_bounds__(kSplitTileWaves * OMH_WAVE)
void proj_split_i8_tile_kernel(const float *__restrict__ x, int64_t ldx, int8_t *__restrict__ xb, int T, int I) {
    __shared__ int s_e[16];
    const int u = blockIdx.x, lane = threadIdx.x % OMH_WAVE, w = threadIdx.x / OMH_WAVE;
    static_assert(kSplitTileWaves == 16, "one token per wave");
    {
        const float *xr = x + (size_t)min(16 * u + w, T - 1) * ldx;   // (padding tokens repeat the last one)
        float m = 0.f;
#pragma unroll 8
        for (int k = 4 * lane; k < I; k += 4 * OMH_WAVE) {
            const float4 v = *reinterpret_cast<const float4 *>(xr + k);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        m = omh_lane_max(m);
        if (lane == 0) s_e[w] = omh_i8_exponent(m);
    }
    __syncthreads();
    const int l16 = lane % 16, g = lane / 16;
    const int t = min(16 * u + l16, T - 1), E = s_e[l16];
    const float *xr = x + (size_t)t * ldx + 16 * g;
    const size_t plane = i8_plane_bytes(T, I);
    int8_t *dst = xb + (size_t)u * 2048 + 16 * lane;
#pragma unroll 2
    for (int j = w; j < I / 64; j += kSplitTileWaves) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = *reinterpret_cast<const float4 *>(xr + 64 * j + 4 * q);
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        v4i a, b, c;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int8_t a4[4], b4[4], c4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) omh_i8_split(v[4 * q + e], E, a4[e], b4[e], c4[e]);
            a[q] = (int)(uint8_t)a4[0] | (int)(uint8_t)a4[1] << 8 | (int)(uint8_t)a4[2] << 16 | (int)((uint32_t)(uint8_t)a4[3] << 24);
            b[q] = (int)(uint8_t)b4[0] | (int)(uint8_t)b4[1] << 8 | (int)(uint8_t)b4[2] << 16 | (int)((uint32_t)(uint8_t)b4[3] << 24);
            c[q] = (int)(uint8_t)c4[0] | (int)(uint8_t)c4[1] << 8 | (int)(uint8_t)c4[2] << 16 | (int)((uint32_t)(uint8_t)c4[3] << 24);
        }
        // fragment (block j / 2, tile u, half j % 2)
        const size_t o = (size_t)(j >> 1) * i8_tiles(T) * 2048 + (j & 1) * 1024;
        *reinterpret_cast<v4i *>(dst + o) = a;
        *reinterpret_cast<v4i *>(dst + plane + o) = b;
        *reinterpret_cast<v4i *>(dst + 2 * plane + o) = c;
    }
    // the token scales, in every block's entry
    const float sc = ldexpf(1.f, s_e[threadIdx.x % 16]);
    float *scl = reinterpret_cast<float *>(xb + kI8Planes * plane);
    for (int i = threadIdx.x; i < 16 * (I / kI8Blk); i += kSplitTileWaves * OMH_WAVE) {
        const int tt = 16 * u + i % 16;
        if (tt < T) scl[(size_t)(i / 16) * T + tt] = sc;
    }
}

constexpr int kI8Rows = 64;                 // rows of a wave's tile

// PT: x has one scale per token (the split kernel's planes): a wave then
// sums each plane exactly in int32 over its whole k range (|sum| <= 2^13 k
// for plane values within [-64, 64]) and combines once at the end.  Else
// (planes written per 128-wide head block by the decode core) the planes
// and the block scale are combined after every block.
template <int G, int TT, bool F32, bool PT>
__global__ __launch_bounds__(4 * OMH_WAVE, 1)
void proj_i8_kernel(const ProjArgs p, int nb, const F32Part f, int nrg, int ntt, int per) {
    constexpr int RW = kI8Rows / 16, NTOK = 16 * TT, NP = kI8Planes;
    constexpr int kTileFloats = kI8Rows * NTOK;
    const int L = blockIdx.x;
    const int ntiles = nrg * ntt;
    if constexpr (F32) {
        if (L >= 8 * per) {
            const int i = L - 8 * per;
            if (i < f.nwg) proj_mfma_wg<1, 1, 8>(f.p, i % f.gx, i / f.gx);
            return;
        }
    }
    const int tile = (L % 8) * per + L / 8;
    if (tile >= ntiles) return;
    const int rg = tile / ntt, tt0 = tile % ntt;
    __shared__ v4f s_red[4][RW][TT][OMH_WAVE];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, gq = lane / 16;
    const int r0 = rg * kI8Rows, t0 = tt0 * NTOK;
    const int g = blockIdx.y;
    const int kb0 = (g * 4 + w) * nb;                      // the wave's first 128-wide block
    const int8_t *X = reinterpret_cast<const int8_t *>(p.xb);
    const size_t plane = i8_plane_bytes(p.T, p.I), bstride = (size_t)i8_tiles(p.T) * 2048;
    const float *scl = reinterpret_cast<const float *>(X + NP * plane);

    const int8_t *wp[RW];
    const int8_t *xp[TT];
    const float *sp[TT];
#pragma unroll
    for (int rw = 0; rw < RW; rw++) wp[rw] = p.Q + (size_t)min(r0 + 16 * rw + l16, p.O - 1) * p.I + 16 * gq;
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int u = min(t0 / 16 + tt, i8_tiles(p.T) - 1);       // token tile
        xp[tt] = X + (size_t)u * 2048 + 16 * lane;
        sp[tt] = scl + min(t0 + 16 * tt + l16, p.T - 1);
    }

    // one block's operands: weights [RW][2 halves], x [TT][NP][2], scales [TT]
    v4i wq[2][RW][2], xq[2][TT][NP][2];
    float sq[2][TT];
    auto load = [&](int kb, auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
#pragma unroll
        for (int rw = 0; rw < RW; rw++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                wq[sl][rw][h] = *reinterpret_cast<const v4i *>(wp[rw] + (size_t)kb * kI8Blk + 64 * h);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
#pragma unroll
            for (int pl = 0; pl < NP; pl++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    xq[sl][tt][pl][h] = *reinterpret_cast<const v4i *>(xp[tt] + pl * plane + kb * bstride + 1024 * h);
            sq[sl][tt] = sp[tt][(size_t)kb * p.T];
        }
    };
    v4f acc[RW][TT];
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[rw][tt] = v4f{0.f, 0.f, 0.f, 0.f};
    v4i ia[PT ? NP : 1][RW][TT];
#pragma unroll
    for (int pl = 0; pl < (PT ? NP : 1); pl++)
#pragma unroll
        for (int rw = 0; rw < RW; rw++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) ia[pl][rw][tt] = v4i{0, 0, 0, 0};
    auto compute = [&](auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
        const v4i zero = {0, 0, 0, 0};
        if constexpr (PT) {
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int rw = 0; rw < RW; rw++)
#pragma unroll
                    for (int pl = 0; pl < NP; pl++)
#pragma unroll
                        for (int h = 0; h < 2; h++)
                            ia[pl][rw][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wq[sl][rw][h], xq[sl][tt][pl][h],
                                                                                   ia[pl][rw][tt], 0, 0, 0);
            return;
        }
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int rw = 0; rw < RW; rw++) {
                v4i a[NP];
#pragma unroll
                for (int pl = 0; pl < NP; pl++) {
                    a[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wq[sl][rw][0], xq[sl][tt][pl][0], zero, 0, 0, 0);
                    a[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wq[sl][rw][1], xq[sl][tt][pl][1], a[pl], 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float lo = (float)(a[1][r] * 128 + a[2][r]);      // |.| <= 2^27: exact in int32
                    const float v = fmaf(lo, 0x1p-14f, (float)a[0][r]);
                    acc[rw][tt][r] = fmaf(v, sq[sl][tt], acc[rw][tt][r]);
                }
            }
    };
    // Two blocks per iteration, one block ahead, every load unconditional
    // (the prefetch past the last block re-loads it): the loop body is
    // straight-line and both edges into the loop header leave the same
    // loads (slot 0) in flight, so the compiler's load-counter waits before
    // each compute cover only that slot's loads instead of draining all.
    const int kl = kb0 + nb - 1;
    load(kb0, std::integral_constant<int, 0>{});
#pragma unroll 1
    for (int b = 0; b < nb; b += 2) {
        __builtin_amdgcn_sched_barrier(0);
        load(min(kb0 + b + 1, kl), std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
        compute(std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        load(min(kb0 + b + 2, kl), std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        compute(std::integral_constant<int, 1>{});
    }

    if constexpr (PT) {
        // the token's scale (the same in every block entry)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const float st = sp[tt][0];
#pragma unroll
            for (int rw = 0; rw < RW; rw++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float lo = fmaf((float)ia[2][rw][tt][r], 0x1p-7f, (float)ia[1][rw][tt][r]);
                    acc[rw][tt][r] = fmaf(lo, 0x1p-7f, (float)ia[0][rw][tt][r]) * st;
                }
        }
    }

    // the workgroup's 4 k-subslices, in wave order; wave w then finishes
    // row tile w
#pragma unroll
    for (int rw = 0; rw < RW; rw++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) s_red[w][rw][tt][lane] = acc[rw][tt];
    __syncthreads();
    v4f y[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
        y[tt] = ((s_red[0][w][tt][lane] + s_red[1][w][tt][lane]) + s_red[2][w][tt][lane]) + s_red[3][w][tt][lane];

    if constexpr (G > 1) {
        float *mine = p.part + ((size_t)tile * G + g) * kTileFloats;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            float *d = mine + ((w * TT + tt) * OMH_WAVE + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; r++) __hip_atomic_store(d + r, y[tt][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);           // this thread's stores are complete
        __syncthreads();
        if (tid == 0) s_last = __hip_atomic_fetch_add(p.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
        __syncthreads();
        if (!s_last) return;
        v4f pt[G][TT];
#pragma unroll
        for (int gg = 0; gg < G; gg++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const float *q = p.part + ((size_t)tile * G + gg) * kTileFloats + ((w * TT + tt) * OMH_WAVE + lane) * 4;
#pragma unroll
                for (int r = 0; r < 4; r++) pt[gg][tt][r] = __hip_atomic_load(q + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            y[tt] = pt[0][tt];
#pragma unroll
            for (int gg = 1; gg < G; gg++) y[tt] += pt[gg][tt];
        }
        if (tid == 0) __hip_atomic_store(p.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // lane holds rows 4gq .. 4gq+3 of row tile w for token l16 of token tile tt
    const int o = r0 + 16 * w + 4 * gq;
    if (o >= p.O) return;
    const float4 sc = *reinterpret_cast<const float4 *>(p.scale + o);
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int t = t0 + 16 * tt + l16;
        if (t >= p.T) continue;
        float4 v;
        v.x = y[tt][0] * sc.x;
        v.y = y[tt][1] * sc.y;
        v.z = y[tt][2] * sc.z;
        v.w = y[tt][3] * sc.w;
        *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) = v;
    }
}

// ------------------------------------ int8 rows, prefill-sized T: GEMM
// For hundreds of tokens and more the projection is a dense contraction
// (the 35B in_proj at T = 4096: 3 x 103 G int8 multiply-adds with x as
// three planes), bound by the int8 matrix cores if operands are reused from
// LDS and registers rather than re-read from L2 by every wave.  A workgroup
// of 8 waves owns a 256-row x 64-token output tile over the whole k range;
// wave (wr, wt) = (w % 4, w / 4) the rows 64 wr .. +63 for the 32 tokens
// 32 wt .. +31 and the three planes: 4 x 2 x 3 accumulators of
// v_mfma_i32_16x16x64_i8, 96 int32 per lane, kept in VGPRs (two waves per
// SIMD).  Per 64-wide k step the workgroup's 16 weight fragments (16 rows x
// 64 k, 16 KiB) and 12 x fragments (4 token tiles x 3 planes, 12 KiB, 1 KiB
// contiguous runs of the i8_off layout) go from L2 / HBM straight into one
// of four LDS stages (buffer loads to LDS, three steps ahead, each fragment
// loaded once, by one wave), and each wave reads its 4 weight and 6 x
// fragments (lane-contiguous 16 bytes: no bank conflicts) one step ahead,
// while the current step's 24 products run.  One barrier per step: before
// it each wave waits for its own copies into the stage the next step reads
// ahead, so a stage is read only once every wave's copies into it have
// landed, and it is refilled only after every wave has passed the barrier
// that follows its last read.  Every sum is exact in int32 (|sum| <= 64 x
// 127 x k < 2^31 for k <= 2^25 / 127); the planes, the token's scale and the
// row scale combine once at the end, as in proj_i8_kernel's per-token form.
// Tiles go to the XCDs by token tile (XCD x takes token tiles x, x + 8, ..),
// each XCD walking patches of 4 row blocks x its token tiles, so the
// workgroups one XCD runs together share their weights and x in its L2.
constexpr int kGmRows = 256, kGmTok = 64;
constexpr int kGmWFrags = kGmRows / 16, kGmXFrags = kI8Planes * kGmTok / 16;   // fragments of one k step
constexpr int kGmStage = (kGmWFrags + kGmXFrags) * 1024;                       // bytes of one LDS stage
constexpr int kGmWgs = 256;                                                    // resident workgroups (one per CU)
#define OMH_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Persistent: workgroup b takes the tiles of blocks b, b + gridDim.x, ...
// (block i: XCD i % 8, the XCD's i / 8-th tile, below), and its copy stream
// runs on across tiles, so the next tile's first steps load while the
// current one finishes and stores its outputs.
__device__ __forceinline__ bool gemm_tile(int i, int nrb, int ntt, int &R0, int &t0) {
    const int xcd = i % 8, j = i / 8;
    const int nx = (ntt - xcd + 7) / 8;                      // token tiles of this XCD
    if (j >= nx * nrb) return false;
    const int grp = j / (4 * nx), rem = j % (4 * nx);
    const int gr = min(4, nrb - 4 * grp);                    // row blocks in this patch
    R0 = (4 * grp + rem % gr) * kGmRows;
    t0 = (xcd + 8 * (rem / gr)) * kGmTok;
    return true;
}

__global__ __launch_bounds__(8 * OMH_WAVE, 1)
void proj_i8_gemm_kernel(const ProjArgs p, int nrb, int ntt) {
    // four stages, separate arrays, so each stage's copies and reads are
    // told apart by the compiler (its waits for this wave's copies into a
    // stage then cover only that stage)
    __shared__ __attribute__((aligned(16))) int8_t s_st0[kGmStage], s_st1[kGmStage], s_st2[kGmStage], s_st3[kGmStage];
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int wr = w % 4, wt = w / 4;
    const int l16 = lane % 16, gq = lane / 16;
    const int S = p.I / 64;                                  // k steps per tile (a multiple of 4)
    const int8_t *X = reinterpret_cast<const int8_t *>(p.xb);
    const size_t plane = i8_plane_bytes(p.T, p.I), bstride = (size_t)i8_tiles(p.T) * 2048;
    const float *scl = reinterpret_cast<const float *>(X + kI8Planes * plane);
    const int G = gridDim.x, b0 = blockIdx.x;
    int NTL = 0;                                             // this workgroup's tiles
    {
        int r, t;
        while (gemm_tile(b0 + G * NTL, nrb, ntt, r, t)) NTL++;
    }
    if (NTL == 0) return;
    const int NG = NTL * S;                                  // k steps over all of its tiles

    // The copies of one step, 4 per wave: weight fragments 2w, 2w + 1 of the
    // tile (rows R0 + 16 f .. +15 at k = 64 s .. +63: one contiguous 1 KiB
    // run of the tiled copy; the step in the scalar offset) and x fragments
    // w and w + 8 (fragment f = 4 plane + token tile; waves 4..7, with no
    // second one, copy their first again).
    const int nrf = (p.O + 15) / 16;                         // 16-row fragments of the tiled weights
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p.Qt), 0, (int)(tile_q8_bytes(p.O, p.I)), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(X), 0, (int)(kI8Planes * plane), 0x00020000);
    int xf[2], xpl[2], xtt[2];
#pragma unroll
    for (int f = 0; f < 2; f++) {
        const int fr = w + 8 * f < kGmXFrags ? w + 8 * f : w;
        xf[f] = kGmWFrags + fr;
        xpl[f] = fr / 4;
        xtt[f] = fr % 4;
    }
    auto stage_of = [&](auto st_c) __attribute__((always_inline)) -> int8_t * {
        constexpr int st = decltype(st_c)::value;
        if constexpr (st == 0) return s_st0;
        else if constexpr (st == 1) return s_st1;
        else if constexpr (st == 2) return s_st2;
        else return s_st3;
    };
    // the next step of the workgroup's copy stream: tile ck, k step cs (past
    // the end: the last step again, unused); the stream runs in order, so the
    // tile's rows and tokens are worked out once per tile
    int ck = 0, cs = 0, cR0 = 0, ct0 = 0;
    gemm_tile(b0, nrb, ntt, cR0, ct0);
    auto copy = [&](auto st_c) __attribute__((always_inline)) {
        int8_t *dst = stage_of(st_c);
        const int R0 = cR0, t0 = ct0, s = cs;
        if (++cs == S) {
            if (ck + 1 < NTL) {
                cs = 0;
                gemm_tile(b0 + G * ++ck, nrb, ntt, cR0, ct0);
            } else {
                cs = S - 1;
            }
        }
        const int xo = (int)((s >> 1) * bstride) + (s & 1) * 1024;
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int wv = min(R0 / 16 + 2 * w + f, nrf - 1) * S * 1024 + 16 * lane;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, OMH_LDS(dst + (2 * w + f) * 1024), 16, wv, 1024 * s, 0, 0);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int xv = (int)(xpl[f] * plane) + min(t0 / 16 + xtt[f], i8_tiles(p.T) - 1) * 2048 + 16 * lane;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, OMH_LDS(dst + xf[f] * 1024), 16, xv, xo, 0, 0);
        }
    };
    v4i fr[2][4 + 2 * kI8Planes];   // [slot][W rows 0..3, x (token tile, plane)]: one step's operands
    // part 0: the weights and token tile 0's x; part 1: token tile 1's x
    auto get = [&](auto st_c, auto slot_c, auto part_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value, part = decltype(part_c)::value;
        const int8_t *st = stage_of(st_c) + 16 * lane;
        if constexpr (part == 0)
#pragma unroll
            for (int rw = 0; rw < 4; rw++) fr[sl][rw] = *reinterpret_cast<const v4i *>(st + (4 * wr + rw) * 1024);
#pragma unroll
        for (int pl = 0; pl < kI8Planes; pl++)
            fr[sl][4 + kI8Planes * part + pl] = *reinterpret_cast<const v4i *>(st + (kGmWFrags + 4 * pl + 2 * wt + part) * 1024);
    };

    v4i acc[kI8Planes][4][2];       // [plane][row fragment][token tile]
    auto zero = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int pl = 0; pl < kI8Planes; pl++)
#pragma unroll
            for (int rw = 0; rw < 4; rw++)
#pragma unroll
                for (int tt = 0; tt < 2; tt++) acc[pl][rw][tt] = v4i{0, 0, 0, 0};
    };
    auto compute = [&](auto slot_c, auto tt_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value, tt = decltype(tt_c)::value;
#pragma unroll
        for (int rw = 0; rw < 4; rw++)
#pragma unroll
            for (int pl = 0; pl < kI8Planes; pl++)
                acc[pl][rw][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fr[sl][rw], fr[sl][4 + kI8Planes * tt + pl],
                                                                        acc[pl][rw][tt], 0, 0, 0);
    };
    // lane holds rows 4gq .. 4gq+3 of row fragment rw for token l16 of token tile tt
    auto store = [&](int k) __attribute__((always_inline)) {
        int R0, t0;
        gemm_tile(b0 + G * k, nrb, ntt, R0, t0);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const int t = t0 + 32 * wt + 16 * tt + l16;
            const float st = scl[min(t, p.T - 1)];         // the token's scale (block 0's entry)
#pragma unroll
            for (int rw = 0; rw < 4; rw++) {
                const int o = R0 + 64 * wr + 16 * rw + 4 * gq;
                if (t >= p.T || o >= p.O) continue;
                const float4 sc4 = *reinterpret_cast<const float4 *>(p.scale + o);
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float lo = fmaf((float)acc[2][rw][tt][r], 0x1p-7f, (float)acc[1][rw][tt][r]);
                    v[r] = fmaf(lo, 0x1p-7f, (float)acc[0][rw][tt][r]) * st;
                }
                *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) =
                    make_float4(v[0] * sc4.x, v[1] * sc4.y, v[2] * sc4.z, v[3] * sc4.w);
            }
        }
    };
    // the wave's copies of all but the last step issued are complete, then
    // every wave's (vmcnt(4): 4 copies per step; other memory operations in
    // flight, the output stores of a finished tile, are older and complete
    // first)
    auto step_barrier = [&]() __attribute__((always_inline)) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0x0F74);                  // vmcnt(4), expcnt / lgkmcnt not waited
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // Step g (stage g % 4, register slot g % 2): the copies of step g + 3 go
    // into stage (g + 3) % 4 (last read during step g - 2, before the barrier
    // that ended step g - 1); step g + 1's operands are read from its stage,
    // whose copies (issued in step g - 2) every wave waited for before that
    // barrier; step g's products run from registers.
    // (The reads of step g + 1 go out in two parts, each before the half of
    // step g's products that follows it, so that no more LDS reads are in
    // flight than the wait counter expresses and the products' waits cover
    // only the previous step's reads.)
    auto step = [&](int g, auto m_c) __attribute__((always_inline)) {
        constexpr int m = decltype(m_c)::value;
        using SN = std::integral_constant<int, (m + 1) % 4>;
        using RN = std::integral_constant<int, (m + 1) % 2>;
        using RC = std::integral_constant<int, m % 2>;
        copy(std::integral_constant<int, (m + 3) % 4>{});        // step g + 3
        get(SN{}, RN{}, std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        compute(RC{}, std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        get(SN{}, RN{}, std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
        compute(RC{}, std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
        step_barrier();
    };
    zero();
    copy(std::integral_constant<int, 0>{});
    copy(std::integral_constant<int, 1>{});
    copy(std::integral_constant<int, 2>{});
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F74);                      // steps 0 and 1 copied (this wave)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    get(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    get(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
#pragma unroll 1
    for (int g = 0; g < NG; g += 4) {
        step(g, std::integral_constant<int, 0>{});
        step(g + 1, std::integral_constant<int, 1>{});
        step(g + 2, std::integral_constant<int, 2>{});
        step(g + 3, std::integral_constant<int, 3>{});
        if ((g + 4) % S == 0) {                              // a tile's last step: its outputs
            store(g / S);
            zero();
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);                      // (the last, unused copies land before the workgroup ends)
}
#undef OMH_LDS

// The GEMM takes int8 rows with x split per token (not the decode core's
// per-head planes) and the tiled copy of the weights, from kGmMinT tokens
// (OMH_I8_GEMM=0 / 1 overrides, for tuning), with k a multiple of the loop
// body's four 64-wide steps.
constexpr int kGmMinT = 256;
bool use_i8_gemm(const ProjArgs &p) {
    if (p.x_split || !p.Qt || p.I % 256 != 0 || p.I > (1 << 25) / 127) return false;
    // (buffer offsets are 32-bit)
    if (tile_q8_bytes(p.O, p.I) >= (1u << 31) || kI8Planes * i8_plane_bytes(p.T, p.I) >= (1u << 31)) return false;
    if (const char *e = getenv("OMH_I8_GEMM")) return e[0] == '1';
    return p.T >= kGmMinT;
}

void launch_i8_gemm(const ProjArgs &p, hipStream_t st) {
    const int nrb = (p.O + kGmRows - 1) / kGmRows, ntt = (p.T + kGmTok - 1) / kGmTok;
    const int per = (ntt + 7) / 8 * nrb;                     // tiles of the XCD with the most
    // one resident workgroup per CU (LDS), each taking every 256th block
    hipLaunchKernelGGL(proj_i8_gemm_kernel, dim3(std::min(8 * per, kGmWgs)), dim3(8 * OMH_WAVE), 0, st, p, nrb, ntt);
}

// Launch shape of the fp32-MFMA projection: one row tile per workgroup (k
// split over its 4 waves) unless that leaves k-slices narrower than a
// 64-wide block or far more workgroups than the device holds at once; a
// few rows (e.g. the fp32 b / a rows beside int8 ones) take one token tile
// per workgroup, so there are more of them.
struct F32Plan {
    int rt, tpw;
    dim3 grid;
};
F32Plan f32_plan(const ProjArgs &p) {
    F32Plan f;
    const int tiles = (p.O + 15) / 16;
    f.tpw = tiles * ((p.T + kMfmaTok - 1) / kMfmaTok) < 64 ? 16 : kMfmaTok;
    const int tb = (p.T + f.tpw - 1) / f.tpw;
    f.rt = 1;
    if (p.I % 256 != 0 || tiles * tb > 4096) f.rt = 2;
    if (p.I % 128 != 0 || tiles * tb > 8192) f.rt = 4;
    f.grid = dim3((tiles + f.rt - 1) / f.rt, tb);
    return f;
}

// Launch plan of the wave-tile kernel for O int8 rows, T tokens, I inputs:
// tokens per wave 16 * TT, with the largest TT (up to what T needs) that
// still gives 768 waves
// (three quarters of the SIMDs); with few rows, TT = 1, and a k split
// over G workgroups only while that leaves fewer than 256 waves (the split
// costs a round trip of partial tiles through memory).  TT = 0: the kernel
// does not take the shape.
struct WvPlan {
    int TT, G;
};
// weight ring depth (blocks ahead) of the wave kernel (deeper rings for the
// narrow token tiles measured no faster: their loop is bound by issue, not
// by load latency)
constexpr int wv_wd(int) { return 2; }
WvPlan q8_wave_plan(int O, int T, int I) {
    WvPlan w{0, 1};
    if (I % (4 * kWvK * 2) != 0) return w;
    const long rg = (O + kWvRows - 1) / kWvRows;
    auto waves = [&](int tt) { return rg * ((T + 16 * tt - 1) / (16 * tt)) * 4; };
    int tt = T <= 16 ? 1 : (T <= 32 ? 2 : 4);     // no wider than the tokens there are
    while (tt > 1 && waves(tt) < 768) tt /= 2;
    // TPT = 16 / tt threads per token share its block sums
    if ((I / 64) % (16 / tt) != 0) return w;
    const int wd = wv_wd(tt);                      // blocks per wave: a multiple of wd
    while (w.G < 8 && waves(tt) * w.G < 256 && I % (4 * kWvK * wd * 2 * w.G) == 0) w.G *= 2;
    if (I % (4 * kWvK * wd * w.G) != 0) return w;
    w.TT = tt;
    return w;
}

template <int TT>
void launch_q8_wave_tt(const ProjArgs &p, int G, int nb, const F32Part &f, bool with, dim3 grid, hipStream_t st) {
    constexpr int WD = wv_wd(TT);
    const dim3 blk(4 * OMH_WAVE);
    if (G == 1 && with) hipLaunchKernelGGL((proj_q8_wave_kernel<1, WD, true, TT>), grid, blk, 0, st, p, nb, f);
    else if (G == 1) hipLaunchKernelGGL((proj_q8_wave_kernel<1, WD, false, TT>), grid, blk, 0, st, p, nb, f);
    else if (G == 2) hipLaunchKernelGGL((proj_q8_wave_kernel<2, WD, false, TT>), grid, blk, 0, st, p, nb, f);
    else if (G == 4) hipLaunchKernelGGL((proj_q8_wave_kernel<4, WD, false, TT>), grid, blk, 0, st, p, nb, f);
    else hipLaunchKernelGGL((proj_q8_wave_kernel<8, WD, false, TT>), grid, blk, 0, st, p, nb, f);
}

// The int8 rows of q by plan w; with f32 (the fp32 rows, n_q = 0) also
// those, in the same launch, when their plan is the one-token-tile shape
// the wave kernel carries (proj_mfma_wg<1, 1, 8>).  *f32_done says whether
// f32 was launched.
void launch_q8_wave(const ProjArgs &p, WvPlan w, const ProjArgs *f32, bool *f32_done, hipStream_t st) {
    const int nb = p.I / (4 * kWvK * w.G);
    F32Part f{};
    f.nrg = (p.O + kWvRows - 1) / kWvRows;
    const int ty = (p.T + 16 * w.TT - 1) / (16 * w.TT);
    bool with = false;
    if (f32 && w.G == 1) {
        const F32Plan fp = f32_plan(*f32);
        with = fp.rt == 1 && fp.tpw == 16 && fp.grid.y > 1 && f32->I / 4 / 64 % 8 == 0;
        if (with) {
            f.p = *f32;
            f.gx = fp.grid.x;
            f.nwg = fp.grid.x * fp.grid.y;
        }
    }
    *f32_done = with;
    const int extra = with ? (f.nwg + ty - 1) / ty : 0;
    const dim3 grid(f.nrg + extra, ty, w.G);
    if (w.TT == 4) launch_q8_wave_tt<4>(p, w.G, nb, f, with, grid, st);
    else if (w.TT == 2) launch_q8_wave_tt<2>(p, w.G, nb, f, with, grid, st);
    else launch_q8_wave_tt<1>(p, w.G, nb, f, with, grid, st);
}

// ---------------------------------------- int8 rows, streaming (T <= 64)
// For decode-sized batches the projection is a stream of the weights from
// HBM (25 MB for the 35B in_proj at 4.6 us), which needs megabytes of loads
// in flight.  A workgroup owns RT row tiles (16 rows each) for all T tokens
// and splits k over its 4 waves (and G workgroups); every wave requests all
// of its weights (RT x NB blocks x 2 halves of 16 bytes per lane) before
// anything else, then walks its k range block by block with x one block
// ahead from L2 (x is per-token scaled: exact int32 sums over the range,
// one fp32 combine at the end).  The grid is about one workgroup per CU.
// PT as for proj_i8_kernel: per-token scales (split kernel) sum in int32 over
// the whole range; per-block scales (planes the decode core wrote per head)
// combine after every block.  The k split G is gridDim.y; the fp32 rows of
// the projection, if any, are the first f.nwg workgroups of row y = 0 (first,
// so they start at once instead of queueing behind the int8 tiles).
template <int RT, int NT, int NB, bool PT>
__global__ __launch_bounds__(4 * OMH_WAVE, 1)
void proj_i8_stream_kernel(const ProjArgs p, const F32Part f) {
    constexpr int NP = kI8Planes;
    constexpr int kTileFloats = RT * 16 * NT * 16;
    const int G = gridDim.y;
    if ((int)blockIdx.x < f.nwg) {
        if (blockIdx.y == 0) proj_mfma_wg<1, 1, 8>(f.p, blockIdx.x % f.gx, blockIdx.x / f.gx);
        return;
    }
    __shared__ v4f s_red[4][RT][NT][OMH_WAVE];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    const int l16 = lane % 16, gq = lane / 16;
    const int rg = blockIdx.x - f.nwg, g = blockIdx.y;
    const int r0 = rg * RT * 16;
    const int kb0 = (g * 4 + w) * NB;                       // the wave's first 128-wide block
    const int8_t *X = reinterpret_cast<const int8_t *>(p.xb);
    const size_t plane = i8_plane_bytes(p.T, p.I), bstride = (size_t)i8_tiles(p.T) * 2048;
    const float *scl = reinterpret_cast<const float *>(X + NP * plane);

    // Every workgroup walks the same x pieces; in the same order they would
    // all hit the same L2 channels at once.  So the walk starts at a
    // workgroup-dependent token tile (rn) and block (rb): register slot nt
    // holds token tile (nt + rn) % NT and slot b block (b + rb) % NB.
    const int rn = rg % NT, rb = (rg / NT) % NB;
    v4i wq[NB][RT][2];
    const int8_t *xp[NT];
    const float *sp[NT];
    int tok[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int u = min((nt + rn) % NT, i8_tiles(p.T) - 1);     // token tile
        tok[nt] = 16 * ((nt + rn) % NT) + l16;
        xp[nt] = X + (size_t)u * 2048 + 16 * lane;
        sp[nt] = scl + min(tok[nt], p.T - 1);
    }
    auto kblock = [&](int b) __attribute__((always_inline)) { return kb0 + (b + rb) % NB; };
    // x in pieces of (block b, token tile nt), q = b NT + nt, in a ring of
    // XR register slots, XR - 1 pieces ahead of the products
    constexpr int NQ = NB * NT, XR = 3;          // (a deeper ring measured no faster)
    v4i xq[XR][NP][2];
    float xs[XR];
    auto x_load = [&](auto qc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value, b = q / NT, nt = q % NT, sl = q % XR;
#pragma unroll
        for (int pl = 0; pl < NP; pl++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                xq[sl][pl][h] = *reinterpret_cast<const v4i *>(xp[nt] + pl * plane + (size_t)kblock(b) * bstride + 1024 * h);
        if constexpr (!PT) xs[sl] = sp[nt][(size_t)kblock(b) * p.T];
    };
    v4i ia[NP][RT][NT];
    v4f acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            acc[rt][nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int pl = 0; pl < NP; pl++) ia[pl][rt][nt] = v4i{0, 0, 0, 0};
        }
    // (planes, rt, nt) combined into acc with scale st
    auto combine = [&](int rt, int nt, float st) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float lo = fmaf((float)ia[2][rt][nt][r], 0x1p-7f, (float)ia[1][rt][nt][r]);
            acc[rt][nt][r] = fmaf(fmaf(lo, 0x1p-7f, (float)ia[0][rt][nt][r]), st, acc[rt][nt][r]);
        }
    };
    // issue order (pinned by scheduling barriers, or the scheduler sinks
    // each load next to its use and the waits drain everything in flight):
    // the first x pieces, then all of the wave's weights block by block,
    // then x XR - 1 pieces ahead of the products.  Loads retire in issue
    // order, so the products of block b wait only for the weights up to b.
    static_for<XR - 1>([&](auto qc) __attribute__((always_inline)) {
        if constexpr (decltype(qc)::value < NQ) x_load(qc);
    });
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int8_t *src = p.Q + (size_t)min(r0 + 16 * rt + l16, p.O - 1) * p.I + (size_t)kblock(b) * kI8Blk + 16 * gq;
#pragma unroll
            for (int h = 0; h < 2; h++) wq[b][rt][h] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(src + 64 * h));
        }
    __builtin_amdgcn_sched_barrier(0);
    static_for<NQ>([&](auto qc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value, b = q / NT, nt = q % NT, sl = q % XR;
        if constexpr (q + XR - 1 < NQ) x_load(std::integral_constant<int, q + XR - 1>{});
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
#pragma unroll
            for (int pl = 0; pl < NP; pl++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    ia[pl][rt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        wq[b][rt][h], xq[sl][pl][h], (PT || h == 1) ? ia[pl][rt][nt] : v4i{0, 0, 0, 0}, 0, 0, 0);
            if constexpr (!PT) combine(rt, nt, xs[sl]);
        }
        __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (PT)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++) combine(rt, nt, sp[nt][0]);
    // the 4 k-subslices in wave order; wave w then finishes tiles w, w+4, ...
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) s_red[w][rt][nt][lane] = acc[rt][nt];
    __syncthreads();
    constexpr int NTILE = RT * NT, PER = (NTILE + 3) / 4;
    v4f y[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int q = w + 4 * j;
        if (q < NTILE)
            y[j] = ((s_red[0][q / NT][q % NT][lane] + s_red[1][q / NT][q % NT][lane]) + s_red[2][q / NT][q % NT][lane]) +
                   s_red[3][q / NT][q % NT][lane];
    }
    if (G > 1) {
        float *mine = p.part + ((size_t)rg * G + g) * kTileFloats;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int q = w + 4 * j;
            if (q >= NTILE) continue;
            float *d = mine + ((size_t)q * OMH_WAVE + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; r++) __hip_atomic_store(d + r, y[j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) s_last = __hip_atomic_fetch_add(p.cnt + rg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
        __syncthreads();
        if (!s_last) return;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int q = w + 4 * j;
            if (q >= NTILE) continue;
            v4f tsum;
            for (int gg = 0; gg < G; gg++) {
                const float *src = p.part + ((size_t)rg * G + gg) * kTileFloats + ((size_t)q * OMH_WAVE + lane) * 4;
                v4f v;
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = __hip_atomic_load(src + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                tsum = gg == 0 ? v : tsum + v;
            }
            y[j] = tsum;
        }
        if (tid == 0) __hip_atomic_store(p.cnt + rg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int q = w + 4 * j;
        if (q >= NTILE) continue;
        const int rt = q / NT, nt = q % NT;
        const int o = r0 + 16 * rt + 4 * gq, t = 16 * ((nt + rn) % NT) + l16;
        if (o >= p.O || t >= p.T) continue;
        const float4 sc = *reinterpret_cast<const float4 *>(p.scale + o);
        float4 v;
        v.x = y[j][0] * sc.x;
        v.y = y[j][1] * sc.y;
        v.z = y[j][2] * sc.z;
        v.w = y[j][3] * sc.w;
        *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) = v;
    }
}

// ------------------------------- int8 rows, decode batches, split queues
// The streaming kernel's waves issue their x pieces after all of their
// weights, and a wave's loads complete in issue order, so its products wait
// for its whole share of the weight stream and then for x one L2 round trip
// per ring slot.  Here the two streams are on different waves: a workgroup
// of 8 waves owns RT 16-row tiles x all (up to 64) tokens over the whole k
// range; waves 4..7 only copy the weights (from the tiled copy, straight into
// an LDS ring of kDqAhead + 2 128-wide blocks, kDqAhead blocks ahead), waves
// 0..3 only load x (token tile w, three int8 planes, from L2 into a register
// ring kDqX blocks ahead) and run the products.  One barrier per block: a
// loader reaches barrier b once its copies of block b have landed, a compute
// wave when it is about to read block b from LDS, which it does while block
// b - 1's products run (so its reads of block b - 2 have completed, and the
// loaders refill that slot next).  Plane sums are exact in int32 over the
// whole k range (per-token scales), combined once at the end.
constexpr int kDqAhead = 8, kDqX = 4;

template <int RT, int NBC>
__global__ __launch_bounds__(8 * OMH_WAVE, 1)
void proj_i8_dq_kernel(const ProjArgs p, const F32Part f) {
    constexpr int NP = kI8Planes, SL = kDqAhead + 2;
    constexpr int WB = RT * 2 * 1024;                        // bytes of one block of the workgroup's weights
    const int tid = threadIdx.x, lane = tid % OMH_WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / OMH_WAVE);
    if ((int)blockIdx.x < f.nwg) {
        if (w < 4) proj_mfma_wg<1, 1, 8>(f.p, blockIdx.x % f.gx, blockIdx.x / f.gx);
        else __syncthreads();                                // (the fp32 workgroup's one barrier)
        return;
    }
    __shared__ __attribute__((aligned(16))) int8_t s_w[SL * WB];
    const int rg = blockIdx.x - f.nwg, r0 = rg * RT * 16;
    const int NB = NBC > 0 ? NBC : p.I / kI8Blk;             // 128-wide blocks
    const int l16 = lane % 16, gq = lane / 16;

    if (w >= 4) {
        // loader: fragment j = 2 rt + h of a block is (row tile rt, k half h);
        // this wave copies fragments (w - 4) and (w - 4) + 4 (where RT > 2)
        constexpr int FPL = RT * 2 / 4 > 0 ? RT * 2 / 4 : 1;      // fragments per loader wave per block
        const int nrf = (p.O + 15) / 16;
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p.Qt), 0, (int)tile_q8_bytes(p.O, p.I), 0x00020000);
        auto copy = [&](int b) __attribute__((always_inline)) {
            const int bb = b;
            int8_t *dst = s_w + (b % SL) * WB;
#pragma unroll
            for (int q = 0; q < FPL; q++) {
                const int j = min((w - 4) + 4 * q, RT * 2 - 1), rt = j / 2, h = j % 2;
                const int vo = min(r0 / 16 + rt, nrf - 1) * (p.I / 64) * 1024 + 16 * lane;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *)(dst + j * 1024),
                                                         16, vo, (2 * bb + h) * 1024, 0, 0);
            }
        };
        for (int b = 0; b < min(kDqAhead, NB); b++) copy(b);
        for (int b = 0; b < NB; b++) {
            asm volatile("" ::: "memory");
            // this wave's copies of block b have landed (those of the later
            // blocks issued so far may be in flight)
            wait_vmcnt<(kDqAhead - 1) * FPL>(min(kDqAhead - 1, NB - 1 - b) * FPL);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (b + kDqAhead < NB) copy(b + kDqAhead);       // into the slot of block b - 2 (its products are issued)
        }
        return;
    }

    // compute wave: token tile w
    const int8_t *X = reinterpret_cast<const int8_t *>(p.xb);
    const size_t plane = i8_plane_bytes(p.T, p.I), bstride = (size_t)i8_tiles(p.T) * 2048;
    const float *scl = reinterpret_cast<const float *>(X + NP * plane);
    const int u = min(w, i8_tiles(p.T) - 1);
    const int8_t *xp = X + (size_t)u * 2048 + 16 * lane;
    // the epilogue's scales, fetched now (they come from HBM: one more
    // round trip at the end otherwise)
    const int t = 16 * w + l16;
    const float st = scl[min(t, p.T - 1)];                   // the token's scale (block 0's entry)
    float4 rsc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int o = r0 + 16 * rt + 4 * gq;
        rsc[rt] = *reinterpret_cast<const float4 *>(p.scale + (o < p.O ? o : 0));
    }
    v4i xq[kDqX][NP][2];
    auto x_load = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
        const size_t o = (size_t)min(b, NB - 1) * bstride;
#pragma unroll
        for (int pl = 0; pl < NP; pl++)
#pragma unroll
            for (int h = 0; h < 2; h++) xq[sl][pl][h] = *reinterpret_cast<const v4i *>(xp + pl * plane + o + 1024 * h);
    };
    v4i ia[NP][RT];
#pragma unroll
    for (int pl = 0; pl < NP; pl++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) ia[pl][rt] = v4i{0, 0, 0, 0};
    // weight fragments of two blocks: block b + 1's are read from LDS while
    // block b's products run (kDqX is even, so b's parity is static)
    v4i wf[2][RT][2];
    auto w_read = [&](int b, auto par_c) __attribute__((always_inline)) {
        constexpr int par = decltype(par_c)::value;
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                        // block b's weights are in LDS
        asm volatile("" ::: "memory");
        const int8_t *src = s_w + (b % SL) * WB + 16 * lane;
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int h = 0; h < 2; h++) wf[par][rt][h] = *reinterpret_cast<const v4i *>(src + (2 * rt + h) * 1024);
        __builtin_amdgcn_sched_barrier(0);                   // (all reads in flight before the products)
    };
    auto block = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(slot_c)::value;
        if (b + 1 < NB) w_read(b + 1, std::integral_constant<int, (sl + 1) % 2>{});
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int pl = 0; pl < NP; pl++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    ia[pl][rt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[sl % 2][rt][h], xq[sl][pl][h], ia[pl][rt], 0, 0, 0);
        // the ring slot just used, kDqX blocks ahead (none past the last
        // block: the epilogue would wait for those loads)
        if (NBC == 0 || b + kDqX < NB) x_load(b + kDqX, slot_c);
    };
    static_for<kDqX>([&](auto sc) __attribute__((always_inline)) { x_load(decltype(sc)::value, sc); });
    w_read(0, std::integral_constant<int, 0>{});
    if constexpr (NBC > 0) {
        // (straight-line code: the x ring's waits count exactly the loads
        // issued after the block's own, which they do not across a loop's
        // back edge)
#pragma unroll
        for (int b = 0; b < NBC; b += kDqX)
            static_for<kDqX>([&](auto sc) __attribute__((always_inline)) { block(b + decltype(sc)::value, sc); });
    } else {
#pragma unroll 1
        for (int b = 0; b < NB; b += kDqX)
            static_for<kDqX>([&](auto sc) __attribute__((always_inline)) { block(b + decltype(sc)::value, sc); });
    }

    // lane holds rows 4gq .. 4gq+3 of row tile rt for token l16 of token tile w
    if (t >= p.T) return;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int o = r0 + 16 * rt + 4 * gq;
        if (o >= p.O) continue;
        const float4 sc = rsc[rt];
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float lo = fmaf((float)ia[2][rt][r], 0x1p-7f, (float)ia[1][rt][r]);
            v[r] = fmaf(lo, 0x1p-7f, (float)ia[0][rt][r]) * st;
        }
        *reinterpret_cast<float4 *>(p.y + (size_t)t * p.ldy + o) = make_float4(v[0] * sc.x, v[1] * sc.y, v[2] * sc.z, v[3] * sc.w);
    }
}

// Taken for 5..64 tokens of x split per token (not the decode core's
// per-head planes) with the tiled weight copy, k a multiple of 128 kDqX and
// the exact-int32 range (OMH_I8_DQ=0 turns it off, for comparison).
constexpr int kDqRT = 4;
bool use_i8_dq(const ProjArgs &p) {
    if (p.T > 64 || p.T <= 4 || p.x_split || !p.Qt || p.I % (kI8Blk * kDqX) != 0 || p.I > (1 << 25) / 127) return false;
    if (const char *e = getenv("OMH_I8_DQ"))
        if (e[0] == '0') return false;
    return true;
}
void launch_i8_dq(const ProjArgs &p, const F32Part &f, hipStream_t st) {
    const int nrg = (p.O + 16 * kDqRT - 1) / (16 * kDqRT);
    const dim3 grid(f.nwg + nrg), blk(8 * OMH_WAVE);
    if (p.I == 16 * kI8Blk) hipLaunchKernelGGL((proj_i8_dq_kernel<kDqRT, 16>), grid, blk, 0, st, p, f);
    else hipLaunchKernelGGL((proj_i8_dq_kernel<kDqRT, 0>), grid, blk, 0, st, p, f);
}

// Plan of the streaming kernel: T <= 64 tokens, RT row tiles per workgroup,
// a k split over G workgroups, NB = 1, 2 or 4 blocks per wave.  Measured at
// the 35B shapes (B = 64, weights from HBM): the launch should fill the
// device in one round of workgroups (one per CU, 256, the fp32-row ones
// included), and a k split or more rows per workgroup only pay where they
// are needed for that.  So: the most workgroups up to 256, then the
// smallest G, then the smallest RT.  rt = 0: not taken.
struct StPlan {
    int rt, nt, nb, G;
};
constexpr int kCUs = 256;
StPlan i8_stream_plan(int O, int T, int I, int nf32) {
    StPlan best{0, 0, 0, 1};
    if (T > 64 || I % (4 * kI8Blk) != 0) return best;
    const int tiles = (O + 15) / 16, nblk = I / kI8Blk, nt = T <= 16 ? 1 : 4;
    long best_wgs = 0;
    for (int G = 1; G <= 8; G *= 2)
        for (int rt = 1; rt <= 4; rt++) {
            const int nb = nblk / (4 * G);
            if (nb * 4 * G != nblk || (nb != 1 && nb != 2 && nb != 4)) continue;
            const long wgs = (long)(tiles + rt - 1) / rt * G + nf32;
            if (wgs > kCUs || wgs <= best_wgs) continue;
            best = StPlan{rt, nt, nb, G};
            best_wgs = wgs;
        }
    return best;
}

template <int RT, int NT, int NB>
void launch_stream_rt(const ProjArgs &p, const F32Part &f, dim3 grid, hipStream_t st) {
    const dim3 blk(4 * OMH_WAVE);
    if (p.x_split) hipLaunchKernelGGL((proj_i8_stream_kernel<RT, NT, NB, false>), grid, blk, 0, st, p, f);
    else hipLaunchKernelGGL((proj_i8_stream_kernel<RT, NT, NB, true>), grid, blk, 0, st, p, f);
}

template <int NT>
void launch_stream_nt(const ProjArgs &p, const StPlan &sp, const F32Part &f, dim3 grid, hipStream_t st) {
#define OMH_ST(RT)                                                             \
    if (sp.nb == 1) launch_stream_rt<RT, NT, 1>(p, f, grid, st);               \
    else if (sp.nb == 2) launch_stream_rt<RT, NT, 2>(p, f, grid, st);          \
    else launch_stream_rt<RT, NT, 4>(p, f, grid, st);
    if (sp.rt == 1) { OMH_ST(1) } else if (sp.rt == 2) { OMH_ST(2) } else if (sp.rt == 3) { OMH_ST(3) } else { OMH_ST(4) }
#undef OMH_ST
}

// The fp32 rows' workgroups beside the int8 ones: their one-token-tile shape
// (proj_mfma_wg<1, 1, 8>) when it applies, else 0.
int f32_beside(const ProjArgs *f32, F32Part *f) {
    if (!f32) return 0;
    const F32Plan fp = f32_plan(*f32);
    if (!(fp.rt == 1 && fp.tpw == 16 && f32->I / 4 / 64 % 8 == 0)) return 0;
    f->p = *f32;
    f->gx = fp.grid.x;
    f->nwg = fp.grid.x * fp.grid.y;
    return f->nwg;
}

void launch_i8_stream(const ProjArgs &p, const StPlan &sp, const F32Part &f, hipStream_t st) {
    const int nrg = ((p.O + 15) / 16 + sp.rt - 1) / sp.rt;
    const dim3 grid(f.nwg + nrg, sp.G);
    if (sp.nt == 1) launch_stream_nt<1>(p, sp, f, grid, st);
    else launch_stream_nt<4>(p, sp, f, grid, st);
}

// Plan of the int8-core kernel for O int8 rows, T tokens, I inputs: tokens
// per wave 16 TT with the largest TT (up to what T needs) that still gives
// kI8Waves waves, then a k split over G workgroups while there are fewer
// than kI8Waves waves and every wave keeps at least two 128-wide blocks.
// TT = 0: the kernel does not take the shape (I not a multiple of 1024).
constexpr int kI8Waves = 1024;
WvPlan i8_plan(int O, int T, int I) {
    WvPlan w{0, 1};
    if (I % (4 * kI8Blk) != 0) return w;
    const long rg = (O + kI8Rows - 1) / kI8Rows;
    auto waves = [&](int tt) { return rg * ((T + 16 * tt - 1) / (16 * tt)) * 4; };
    int tt = T <= 16 ? 1 : 2;                     // (a 64-token tile needs more registers than a wave has)
    while (tt > 1 && waves(tt) < kI8Waves) tt /= 2;
    // (a wave's k range is an even number of 128-wide blocks: I % (1024 G) == 0)
    if (I % (8 * kI8Blk) != 0) return w;
    while (w.G < 8 && waves(tt) * w.G < kI8Waves && I % (8 * kI8Blk * 2 * w.G) == 0) w.G *= 2;
    w.TT = tt;
    return w;
}

// The projection variant for int8 rows with T > 4: the int8-core kernel
// where it takes the shape, else the bf16 x 3 kernels.
bool use_i8(int T, int I, int n_q) {
    return n_q > 0 && T > 4 && i8_plan(n_q, T, I).TT != 0;
}

template <int TT, bool PT>
void launch_i8_tt(const ProjArgs &p, int G, int nb, const F32Part &f, bool with, dim3 grid, int nrg, int ntt,
                  int per, hipStream_t st) {
    const dim3 blk(4 * OMH_WAVE);
    if (G == 1 && with) hipLaunchKernelGGL((proj_i8_kernel<1, TT, true, PT>), grid, blk, 0, st, p, nb, f, nrg, ntt, per);
    else if (G == 1) hipLaunchKernelGGL((proj_i8_kernel<1, TT, false, PT>), grid, blk, 0, st, p, nb, f, nrg, ntt, per);
    else if (G == 2) hipLaunchKernelGGL((proj_i8_kernel<2, TT, false, PT>), grid, blk, 0, st, p, nb, f, nrg, ntt, per);
    else if (G == 4) hipLaunchKernelGGL((proj_i8_kernel<4, TT, false, PT>), grid, blk, 0, st, p, nb, f, nrg, ntt, per);
    else hipLaunchKernelGGL((proj_i8_kernel<8, TT, false, PT>), grid, blk, 0, st, p, nb, f, nrg, ntt, per);
}

// The int8 rows of q by plan w; with f32 (the fp32 rows, n_q = 0) also
// those, in the same launch, when they take the one-token-tile fp32 shape.
void launch_i8(const ProjArgs &p, WvPlan w, const ProjArgs *f32, bool *f32_done, hipStream_t st) {
    const int nb = p.I / (4 * kI8Blk * w.G);
    const int nrg = (p.O + kI8Rows - 1) / kI8Rows, ntt = (p.T + 16 * w.TT - 1) / (16 * w.TT);
    const int per = (nrg * ntt + 7) / 8;
    F32Part f{};
    bool with = false;
    if (f32 && w.G == 1) {
        const F32Plan fp = f32_plan(*f32);
        with = fp.rt == 1 && fp.tpw == 16 && fp.grid.y > 1 && f32->I / 4 / 64 % 8 == 0;
        if (with) {
            f.p = *f32;
            f.gx = fp.grid.x;
            f.nwg = fp.grid.x * fp.grid.y;
        }
    }
    *f32_done = with;
    const dim3 grid(8 * per + (with ? f.nwg : 0), w.G);
    // per-token scales unless the decode core wrote the planes (per head);
    // the int32 sums stay in range for a wave's k range up to 1024 (2^23)
    const bool pt = !p.x_split && p.I / (4 * w.G) <= 1024;
    if (w.TT == 2 && pt) launch_i8_tt<2, true>(p, w.G, nb, f, with, grid, nrg, ntt, per, st);
    else if (w.TT == 2) launch_i8_tt<2, false>(p, w.G, nb, f, with, grid, nrg, ntt, per, st);
    else if (pt) launch_i8_tt<1, true>(p, w.G, nb, f, with, grid, nrg, ntt, per, st);
    else launch_i8_tt<1, false>(p, w.G, nb, f, with, grid, nrg, ntt, per, st);
}

inline bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

struct XbLayout {
    size_t part, cnt, total;   // byte offsets of the partial tiles and counters, total bytes
    WvPlan w;
    int ncnt;
};
XbLayout xb_layout(int T, int I, int n_q) {
    XbLayout l{};
    const bool i8 = use_i8(T, I, n_q);
    const size_t planes = i8 ? i8_planes_bytes(T, I)
                             : (size_t)3 * T * I * sizeof(uint16_t) + (size_t)T * (I / 64) * sizeof(float);
    l.w = n_q > 0 ? (i8 ? i8_plan(n_q, T, I) : q8_wave_plan(n_q, T, I)) : WvPlan{0, 1};
    l.part = (planes + 255) / 256 * 256;
    // k-split partial tiles and arrival counters: enough for whichever
    // kernel the launch picks (the wave kernel's plan, or the streaming one)
    size_t npart = 0, ncnt = 0;
    if (l.w.TT > 0 && l.w.G > 1) {
        const int ntok = 16 * l.w.TT;
        const size_t tiles = (size_t)((n_q + kWvRows - 1) / kWvRows) * ((T + ntok - 1) / ntok);
        npart = tiles * l.w.G * kWvRows * ntok * sizeof(float);
        ncnt = tiles;
    }
    if (i8)
        for (int nf32 : {0, 16}) {          // (the plan may differ with fp32-row workgroups beside)
            const StPlan sp = i8_stream_plan(n_q, T, I, nf32);
            if (sp.rt > 0 && sp.G > 1) {
                const size_t tiles = (size_t)(((n_q + 15) / 16 + sp.rt - 1) / sp.rt);
                npart = std::max(npart, tiles * sp.G * (size_t)(sp.rt * 16 * sp.nt * 16) * sizeof(float));
                ncnt = std::max(ncnt, tiles);
            }
        }
    l.cnt = l.part + npart;
    l.ncnt = (int)ncnt;
    l.total = l.cnt + ncnt * sizeof(int);
    return l;
}

template <int RG, int KS>
void launch_q8(const ProjArgs &p, hipStream_t st) {
    constexpr int TT = kQ8Tok / 16;
    const dim3 grid((p.O + RG * kQ8Rows - 1) / (RG * kQ8Rows), (p.T + kQ8Tok - 1) / kQ8Tok);
    const int nb = p.I / KS / kQ8K;
    const dim3 blk(4 * OMH_WAVE);
    switch (nb) {
    case 1: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 1, 1>), grid, blk, 0, st, p); break;
    case 2: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 2, 2>), grid, blk, 0, st, p); break;
    case 4: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 4, 4>), grid, blk, 0, st, p); break;
    case 8: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 4, 8>), grid, blk, 0, st, p); break;
    case 16: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 4, 16>), grid, blk, 0, st, p); break;
    case 32: hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 4, 32>), grid, blk, 0, st, p); break;
    default:
        if (nb % 4 == 0) hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 4, 0>), grid, blk, 0, st, p);
        else if (nb % 2 == 0) hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 2, 0>), grid, blk, 0, st, p);
        else hipLaunchKernelGGL((proj_q8_bf16x3_kernel<RG, KS, TT, 1, 0>), grid, blk, 0, st, p);
    }
}

// Row-major int8 weights [O][I] -> the tiled copy (tile_q8_bytes): one
// thread per 16-byte piece of the copy.
__global__ __launch_bounds__(256)
void tile_q8_kernel(const int8_t *__restrict__ Q, int O, int I, int8_t *__restrict__ Qt) {
    const size_t P = (size_t)blockIdx.x * 256 + threadIdx.x;           // piece of the copy
    const int nks = I / 64;
    if (P >= (size_t)(O + 15) / 16 * nks * OMH_WAVE) return;
    const size_t frag = P / OMH_WAVE;
    const int L = (int)(P % OMH_WAVE), rb = (int)(frag / nks), ks = (int)(frag % nks);
    const int o = 16 * rb + L % 16, k = 64 * ks + 16 * (L / 16);
    v4i v = {0, 0, 0, 0};
    if (o < O) v = *reinterpret_cast<const v4i *>(Q + (size_t)o * I + k);
    *reinterpret_cast<v4i *>(Qt + 16 * P) = v;
}

}  // namespace

bool tile_q8_wanted(int O, int I) { return O > 0 && I % 256 == 0 && tile_q8_bytes(O, I) < (1u << 31); }
hipError_t tile_q8(const int8_t *Q, int O, int I, int8_t *Qt, hipStream_t st) {
    if (!tile_q8_wanted(O, I)) return hipErrorInvalidValue;
    const size_t pieces = (size_t)(O + 15) / 16 * (I / 64) * OMH_WAVE;
    hipLaunchKernelGGL(tile_q8_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st, Q, O, I, Qt);
    return hipGetLastError();
}

bool proj_supported(int I, int n_q) { return I >= 64 && I % 64 == 0 && n_q % 16 == 0; }

size_t proj_xb_bytes(int T, int I, int n_q) { return xb_layout(T, I, n_q).total; }

bool proj_x_int8_planes(int T, int I, int n_q) { return use_i8(T, I, n_q); }

hipError_t launch_proj(const ProjArgs &p, hipStream_t st) {
    if (p.O <= 0 || p.T <= 0) return hipSuccess;
    if (!proj_supported(p.I, p.n_q)) return hipErrorInvalidValue;
    // the deferred gated norm: the GEMV's int8 rows only, heads of whole 16-input pieces
    if (p.gssq && (p.T > 4 || p.n_q != p.O || p.gvd < 16 || p.gvd % 16 != 0 || p.I % p.gvd != 0 || !al16(p.gssq)))
        return hipErrorInvalidValue;
    if (p.T <= 4) {
        // k-slices: as many 1024-wide chunks as there are, up to 4 per row group
        const int ks = p.I >= 4096 ? 4 : (p.I >= 2048 ? 2 : 1);
        const int rows_per_wg = (4 / ks) * kGemvRows;
        const int nwg8 = (p.n_q + rows_per_wg - 1) / rows_per_wg, nf = (p.O - p.n_q + 3) / 4;
        const dim3 grid(nwg8 + nf), blk(4 * OMH_WAVE);
#define OMH_GEMV_KS(NT, GN)                                                                                       \
    if (ks == 4) hipLaunchKernelGGL((proj_gemv_kernel<NT, 4, kGemvRows, GN>), grid, blk, 0, st, p, nwg8);         \
    else if (ks == 2) hipLaunchKernelGGL((proj_gemv_kernel<NT, 2, kGemvRows, GN>), grid, blk, 0, st, p, nwg8);    \
    else hipLaunchKernelGGL((proj_gemv_kernel<NT, 1, kGemvRows, GN>), grid, blk, 0, st, p, nwg8);
#define OMH_GEMV(NT)                                                                                              \
    if (p.gssq) { OMH_GEMV_KS(NT, true) } else { OMH_GEMV_KS(NT, false) }
        switch (p.T) {
        case 1: OMH_GEMV(1) break;
        case 2: OMH_GEMV(2) break;
        case 3: OMH_GEMV(3) break;
        default: OMH_GEMV(4) break;
        }
#undef OMH_GEMV
#undef OMH_GEMV_KS
        return hipGetLastError();
    }
    // int8 rows on the bf16 matrix cores (bf16 x 3), the fp32 rows after
    if (p.n_q > 0 && p.xb && p.I % kQ8K == 0 && al16(p.x) && al16(p.y) && p.ldx % 4 == 0 && p.ldy % 4 == 0) {
        const XbLayout lay = xb_layout(p.T, p.I, p.n_q);
        if (lay.total > p.xb_n) return hipErrorInvalidValue;
        ProjArgs q = p;
        q.O = p.n_q;
        q.part = reinterpret_cast<float *>(reinterpret_cast<char *>(p.xb) + lay.part);
        // the caller's always-zero counters where they suffice, else counters
        // in the scratch, cleared by the split launch (or a launch of its own)
        const bool own = p.counters && lay.ncnt <= p.ncounters;
        q.cnt = own ? p.counters : reinterpret_cast<int *>(reinterpret_cast<char *>(p.xb) + lay.cnt);
        const int nclear = own ? 0 : lay.ncnt;
        const bool i8 = use_i8(p.T, p.I, p.n_q);
        // (planes written by the decode core: no split, unless counters need clearing)
        if (i8 && !p.x_split && p.T > 64) {
            hipLaunchKernelGGL(proj_split_i8_tile_kernel, dim3((unsigned)i8_tiles(p.T)), dim3(kSplitTileWaves * OMH_WAVE), 0, st, p.x, p.ldx,
                               reinterpret_cast<int8_t *>(p.xb), p.T, p.I);
            if (nclear > 0)
                hipLaunchKernelGGL(proj_split_i8_kernel, dim3(1), dim3(256), 0, st, p.x, p.ldx,
                                   reinterpret_cast<int8_t *>(p.xb), 0, p.I, q.cnt, nclear);
        } else if (i8 && !p.x_split) {
            hipLaunchKernelGGL(proj_split_i8_kernel, dim3((unsigned)p.T), dim3(256), 0, st, p.x, p.ldx,
                               reinterpret_cast<int8_t *>(p.xb), p.T, p.I, q.cnt, nclear);
        } else if (i8 && nclear > 0) {
            hipLaunchKernelGGL(proj_split_i8_kernel, dim3(1), dim3(256), 0, st, p.x, p.ldx,
                               reinterpret_cast<int8_t *>(p.xb), 0, p.I, q.cnt, nclear);
        } else if (!i8 && (!p.x_split || nclear > 0)) {
            const size_t n8 = (size_t)p.T * (p.I / 8);
            hipLaunchKernelGGL(proj_split_x_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, p.x, p.ldx, p.xb,
                               p.T, p.I, q.cnt, nclear);
        }
        ProjArgs f = p;
        f.y = p.y + p.n_q;
        f.O = p.O - p.n_q;
        f.n_q = 0;
        f.Q = nullptr;
        f.scale = nullptr;
        bool f32_done = false;
        const bool done = lay.w.TT > 0;
        F32Part fs{};
        const int nf32 = i8 ? f32_beside(p.O > p.n_q ? &f : nullptr, &fs) : 0;
        const StPlan sp = i8 ? i8_stream_plan(q.O, p.T, p.I, nf32) : StPlan{0, 0, 0, 1};
        if (i8 && use_i8_dq(q)) {
            launch_i8_dq(q, fs, st);
            f32_done = nf32 > 0;
        } else if (sp.rt > 0) {
            launch_i8_stream(q, sp, fs, st);
            f32_done = nf32 > 0;
        } else if (i8 && use_i8_gemm(q)) launch_i8_gemm(q, st);
        else if (done && i8) launch_i8(q, lay.w, p.O > p.n_q ? &f : nullptr, &f32_done, st);
        else if (done) launch_q8_wave(q, lay.w, p.O > p.n_q ? &f : nullptr, &f32_done, st);
        if (!done) {
            // enough workgroups for the device (a k split where rows are few)
            const int tb = (p.T + kQ8Tok - 1) / kQ8Tok;
            const int rb = (q.O + kQ8Rows - 1) / kQ8Rows;       // row blocks of one wave
            if (rb / 4 * tb >= 128 || p.I % (2 * kQ8K) != 0) launch_q8<4, 1>(q, st);
            else launch_q8<2, 2>(q, st);
        }
        if (p.O == p.n_q || f32_done) return hipGetLastError();
        return launch_proj(f, st);
    }
    const F32Plan fp = f32_plan(p);
    if (fp.rt == 4) launch_mfma_rt<4>(p, fp.grid, fp.tpw, st);
    else if (fp.rt == 2) launch_mfma_rt<2>(p, fp.grid, fp.tpw, st);
    else launch_mfma_rt<1>(p, fp.grid, fp.tpw, st);
    return hipGetLastError();
}

}  // namespace omh
