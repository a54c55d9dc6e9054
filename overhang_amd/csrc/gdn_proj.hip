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
#include <type_traits>

namespace omh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

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
// A workgroup is 4 waves = RG row groups of kGemvRows rows x KS k-slices;
// each wave covers its k-slice in chunks of 1024 (16 per lane).
constexpr int kGemvRows = 8;

// Sum of v[i] over the 64 lanes for 8 values at once, halving the set at
// each of the first three exchanges: lane L ends with the total of value
// 4*bit5(L) + 2*bit4(L) + bit3(L).
__device__ __forceinline__ float sum8_over_lanes(const float (&v)[8], int lane) {
    float u[4], t[2];
    const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float send = h5 ? v[i] : v[i + 4];
        u[i] = (h5 ? v[i + 4] : v[i]) + __shfl_xor(send, 32, OMH_WAVE);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float send = h4 ? u[i] : u[i + 2];
        t[i] = (h4 ? u[i + 2] : u[i]) + __shfl_xor(send, 16, OMH_WAVE);
    }
    float r = (h3 ? t[1] : t[0]) + __shfl_xor(h3 ? t[0] : t[1], 8, OMH_WAVE);
    r += __shfl_xor(r, 4, OMH_WAVE);
    r += __shfl_xor(r, 2, OMH_WAVE);
    r += __shfl_xor(r, 1, OMH_WAVE);
    return r;
}

template <int NT, bool Q8, int KS>
__device__ __forceinline__ void gemv_rows(const ProjArgs &p, int r0, int ks, int lane, float (*red)[NT][OMH_WAVE],
                                          int rg, bool store) {
    float acc[kGemvRows][NT];
#pragma unroll
    for (int i = 0; i < kGemvRows; i++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[i][t] = 0.f;
    const int nrow = min(kGemvRows, p.O - r0);
    const int klen = p.I / KS;
    for (int kc = ks * klen; kc < (ks + 1) * klen; kc += 16 * OMH_WAVE) {
        const int k = kc + 16 * lane;
        if (k < (ks + 1) * klen) {
            WFrag<Q8> wf[kGemvRows];                 // every row's weights in flight together
#pragma unroll
            for (int i = 0; i < kGemvRows; i++) wf[i].load(p, r0 + min(i, nrow - 1), k);
            float x[NT][16];
#pragma unroll
            for (int t = 0; t < NT; t++) load_x16(p.x + (size_t)t * p.ldx + k, x[t]);
#pragma unroll
            for (int i = 0; i < kGemvRows; i++) {
                float w[16];
                wf[i].unpack(w);
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][t] = fmaf(x[t][e], w[e], acc[i][t]);
            }
        }
    }
    // lane L holds row 4*bit5(L) + 2*bit4(L) + bit3(L) after the reduction
    const int myrow = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
    float tot[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = acc[i][t];
        tot[t] = sum8_over_lanes(v, lane);
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
    if (store && (lane & 7) == 0 && myrow < nrow) {
        const int o = r0 + myrow;
        const float sc = Q8 ? p.scale[o] : 1.f;
#pragma unroll
        for (int t = 0; t < NT; t++) p.y[(size_t)t * p.ldy + o] = tot[t] * sc;
    }
}

template <int NT, int KS>
__global__ __launch_bounds__(4 * OMH_WAVE)
void proj_gemv_kernel(const ProjArgs p) {
    constexpr int RG = 4 / KS;
    __shared__ float red[KS > 1 ? (KS - 1) * 4 : 1][NT][OMH_WAVE];
    const int lane = threadIdx.x % OMH_WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / OMH_WAVE);
    const int rg = wv % RG, ks = wv / RG;
    // a row group past the end works on the last group instead (the
    // workgroup stays together for the k-slice reduction) and stores nothing
    const int rs = (blockIdx.x * RG + rg) * kGemvRows;
    const int r0 = min(rs, ((p.O - 1) / kGemvRows) * kGemvRows);
    if (r0 < p.n_q) gemv_rows<NT, true, KS>(p, r0, ks, lane, red, rg, rs < p.O);
    else gemv_rows<NT, false, KS>(p, r0, ks, lane, red, rg, rs < p.O);
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
        if (r0 < p.n_q) mfma_tiles<TT, true, PF>(p, r0, t0, kbeg, klen, lane, acc);
        else mfma_tiles<TT, false, (PF > 2 ? 2 : PF)>(p, r0, t0, kbeg, klen, lane, acc);
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

template <int RT, int TT, int PF>
__global__ __launch_bounds__(4 * OMH_WAVE)
void proj_mfma_kernel(const ProjArgs p) {
    proj_mfma_wg<RT, TT, PF>(p, blockIdx.x, blockIdx.y);
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

inline bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

struct XbLayout {
    size_t part, cnt, total;   // byte offsets of the partial tiles and counters, total bytes
    WvPlan w;
    int ncnt;
};
XbLayout xb_layout(int T, int I, int n_q) {
    XbLayout l{};
    const size_t planes = (size_t)3 * T * I * sizeof(uint16_t) + (size_t)T * (I / 64) * sizeof(float);
    l.w = n_q > 0 ? q8_wave_plan(n_q, T, I) : WvPlan{0, 1};
    const int ntok = 16 * (l.w.TT > 0 ? l.w.TT : 1);
    const size_t tiles = (size_t)((n_q + kWvRows - 1) / kWvRows) * ((T + ntok - 1) / ntok);
    l.part = (planes + 255) / 256 * 256;
    const bool split = l.w.TT > 0 && l.w.G > 1;
    const size_t npart = split ? tiles * l.w.G * kWvRows * ntok * sizeof(float) : 0;
    l.cnt = l.part + npart;
    l.ncnt = split ? (int)tiles : 0;
    l.total = l.cnt + (size_t)l.ncnt * sizeof(int);
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

}  // namespace

bool proj_supported(int I, int n_q) { return I >= 64 && I % 64 == 0 && n_q % 16 == 0; }

size_t proj_xb_bytes(int T, int I, int n_q) { return xb_layout(T, I, n_q).total; }

hipError_t launch_proj(const ProjArgs &p, hipStream_t st) {
    if (p.O <= 0 || p.T <= 0) return hipSuccess;
    if (!proj_supported(p.I, p.n_q)) return hipErrorInvalidValue;
    if (p.T <= 4) {
        // k-slices: as many 1024-wide chunks as there are, up to 4 per row group
        const int ks = p.I >= 4096 ? 4 : (p.I >= 2048 ? 2 : 1);
        const int rows_per_wg = (4 / ks) * kGemvRows;
        const dim3 grid((p.O + rows_per_wg - 1) / rows_per_wg), blk(4 * OMH_WAVE);
#define OMH_GEMV(NT)                                                                        \
    if (ks == 4) hipLaunchKernelGGL((proj_gemv_kernel<NT, 4>), grid, blk, 0, st, p);       \
    else if (ks == 2) hipLaunchKernelGGL((proj_gemv_kernel<NT, 2>), grid, blk, 0, st, p);  \
    else hipLaunchKernelGGL((proj_gemv_kernel<NT, 1>), grid, blk, 0, st, p);
        switch (p.T) {
        case 1: OMH_GEMV(1) break;
        case 2: OMH_GEMV(2) break;
        case 3: OMH_GEMV(3) break;
        default: OMH_GEMV(4) break;
        }
#undef OMH_GEMV
        return hipGetLastError();
    }
    // int8 rows on the bf16 matrix cores (bf16 x 3), the fp32 rows after
    if (p.n_q > 0 && p.xb && p.I % kQ8K == 0 && al16(p.x) && al16(p.y) && p.ldx % 4 == 0 && p.ldy % 4 == 0) {
        const XbLayout lay = xb_layout(p.T, p.I, p.n_q);
        if (lay.total > p.xb_n) return hipErrorInvalidValue;
        ProjArgs q = p;
        q.O = p.n_q;
        q.part = reinterpret_cast<float *>(reinterpret_cast<char *>(p.xb) + lay.part);
        q.cnt = reinterpret_cast<int *>(reinterpret_cast<char *>(p.xb) + lay.cnt);
        // (planes written by the decode core: no split, unless counters need clearing)
        if (!p.x_split || lay.ncnt > 0) {
            const size_t n8 = (size_t)p.T * (p.I / 8);
            hipLaunchKernelGGL(proj_split_x_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, p.x, p.ldx, p.xb,
                               p.T, p.I, q.cnt, lay.ncnt);
        }
        ProjArgs f = p;
        f.y = p.y + p.n_q;
        f.O = p.O - p.n_q;
        f.n_q = 0;
        f.Q = nullptr;
        f.scale = nullptr;
        bool f32_done = false;
        const bool done = lay.w.TT > 0;
        if (done) launch_q8_wave(q, lay.w, p.O > p.n_q ? &f : nullptr, &f32_done, st);
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
