// omh_internal.h — interface between the C-ABI layer (om_hip.hip) and the
// kernel launchers.  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omh {

// Conv history ring: every channel keeps kConvRing slots, and token n of a
// sequence (counted from the last reset or state_set) sits in slot
// n mod kConvRing.  At phase p (= tokens consumed, mod kConvRing) the K-1
// history values, oldest first, are in slots (p + kConvRing+1 - K + j) mod
// kConvRing and slot p is free.  Consuming a token writes it into the free
// slot and advances p; no other slot changes, so readers of the history
// slots never race with the writer.  Slot-major layout
// [seq][kConvRing][conv_dim]: one slot of consecutive channels is one
// contiguous run, so a token reads K-1 values and writes one per channel,
// all in whole lines.
constexpr int kConvRing = 4;          // supports conv kernels K = 2..4

__host__ __device__ inline int ring_slot(int p, int K, int j) {
    return (p + kConvRing + 1 - K + j) & (kConvRing - 1);
}
// Offset of slot `slot` of channel ch for sequence seq.
__host__ __device__ inline size_t ring_at(int seq, int slot, int ch, int conv_dim) {
    return ((size_t)seq * kConvRing + slot) * conv_dim + ch;
}
// Element j (0..3) of a float4.
__host__ __device__ inline float f4_get(const float4 &v, int j) {
    return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}
__host__ __device__ inline void f4_set(float4 &v, int j, float x) {
    if (j == 0) v.x = x; else if (j == 1) v.y = x; else if (j == 2) v.z = x; else v.w = x;
}

// Device pointers of one layer's core weights and state.  The per-sequence
// ring phase is double-buffered by launch parity (epoch): a decode launch
// reads phase[epoch][b] and writes phase[1-epoch][b], and the host flips
// the layer's epoch after enqueueing it.
struct LayerPtrs {
    const float *conv_w;   // [conv_dim][kConvRing], taps right-aligned: zeros, then taps 0..K-1
    const float *A_log;    // [vh]
    const float *dt_bias;  // [vh]
    const float *gnorm;    // [vd]
    float *conv_st;        // [max_seqs][kConvRing][conv_dim] ring
    float *S;              // [max_seqs][vh][kd][vd]
    int *phase;            // [2][max_seqs]
    float *o_raw;          // [max_seqs][vh][vd]   cross-slice gated-norm scratch
    float *ssq;            // [max_seqs][vh][kMaxSlices]
    int *cnt;              // [max_seqs][vh]  arrivals (reset to 0 by the last)
    int epoch, max_seqs;
};
constexpr int kMaxSlices = 8;

// Decode-core launch: nl layers x B sequences (b0 .. b0+B-1), one token each.
constexpr int kMaxDecodeLayers = 32;
// Token t = l*B + b reads qkv + t*ld_qkv, z + t*ld_z, a + t*ld_ab, b + t*ld_ab
// and writes core + t*vh*vd.
struct DecodeArgs {
    const float *qkv;   // [nl*B] rows of >= conv_dim
    const float *z;     // [nl*B] rows of >= vh*vd
    const float *a;     // [nl*B] rows of >= vh
    const float *b;     // [nl*B] rows of >= vh
    float *core;        // [nl][B][vh*vd]
    int64_t ld_qkv, ld_z, ld_ab;
    int B, nl, kh, vh, K;
    float eps;
    int rep;            // vh / kh
    int b0;             // token row b is sequence (state slot) b0 + b
    uint16_t *xb;       // or null; with nl = 1, the core output also as the out_proj scratch's x: bf16 planes and block sums (xpiece) or, with xb_i8, int8 planes and block scales (i8_off); I = vh*vd
    int xb_T, xb_t0;    // the planes' token count, and the planes' token of row 0 of this launch
    bool xb_i8;
    float *ssq_out;     // or null; with 4 column slices and nl = 1: each slice writes o * gnorm * silu(z) of its
                        // columns to core and its sum of squares of o to ssq_out[(b * vh + h) * 4 + slice]; the
                        // norm's 1 / rms is left to the consumer (ProjArgs::gssq)
    LayerPtrs L[kMaxDecodeLayers];
};

// Layout of the bf16 planes of x (the int8 projections' scratch, x as
// hi + mid + lo): per plane, 32-value chunks [I / 32][T][32].  Chunk 4c + s
// of token t holds, at position 8g + j, the value at k = 128c + 32g + 8s + j
// (g < 4, j < 8): exactly what lane group g of a 16-token MFMA operand
// reads in step s of 128-wide k superblock c (the k order both operands
// share: lane group g of a weight fragment then holds 32 consecutive k of
// its row, two 16-byte loads that together cover whole 128-byte lines).
// So 16 tokens' operand for one step is one contiguous 1 KiB run, and every
// 16-byte piece of 8 consecutive k is contiguous.  Element offset of the
// piece holding k = 8m .. 8m+7 of token t (planes of T * I elements each,
// then fp32 sums [T][I / 64]).  A trailing 64-wide block (I % 128 == 64)
// takes the last two chunks, in the 64-wide form of the same order.
__host__ __device__ inline size_t xpiece(int m, int t, int T, int I) {
    const int full = I / 128, c = m / 16;
    if (c < full) return ((size_t)(4 * c + m % 4) * T + t) * 32 + 8 * ((m % 16) / 4);
    return ((size_t)(4 * full + m % 2) * T + t) * 32 + 8 * ((m % 8) / 2);
}

// Layout of x as int8 planes (the scratch of the int8 projections on the
// int8 matrix cores).  Per token t and 128-wide k block b, with the power of
// two 2^E[b][t] (E = ilogb(m) - 5 for the max |x| m over the block, or over
// the token's whole row when one scale serves the row, so every plane value
// lies in [-64, 64]):
//     x = 2^E (p1 + p2 2^-7 + p3 2^-14) + r,   |r| <= 2^(E-15) <= 2^-20 m
// (each step of the split is exact in fp32: omh_i8_split).  Each plane is
// stored in MFMA operand order: the 16-token x 64-k operand of one
// v_mfma_i32_16x16x64_i8 (block b, token tile u = t / 16, half h of the
// block) is one contiguous 1 KiB run in lane order, lane l16 + 16 g holding
// token 16u + l16 at k = 128b + 64h + 16g .. +15 (a wave's load of it is one
// contiguous 1 KiB request).  Token tiles are padded to 16 (padding never
// read into a result that is kept).  Plane p starts at byte p * i8_plane_bytes;
// after the planes, the scales 2^E as fp32 [I/128][T].
constexpr int kI8Blk = 128;
constexpr int kI8Planes = 3;
__host__ __device__ inline int i8_tiles(int T) { return (T + 15) / 16; }
__host__ __device__ inline size_t i8_plane_bytes(int T, int I) { return (size_t)i8_tiles(T) * 16 * I; }
__host__ __device__ inline size_t i8_off(int k, int t, int T) {
    return ((((size_t)(k / kI8Blk) * i8_tiles(T) + t / 16) * 2 + (k % kI8Blk) / 64) * 4 + (k % 64) / 16) * 256 +
           (t % 16) * 16 + k % 16;
}
__host__ __device__ inline size_t i8_planes_bytes(int T, int I) {
    return (size_t)kI8Planes * i8_plane_bytes(T, I) + (size_t)(I / kI8Blk) * T * sizeof(float);
}

// y[t][o] = sum_i x[t][i] * W[o][i] for t < T, o < O.  Rows o < n_q come
// from the int8 matrix Q (times scale[o]); rows o >= n_q from the fp32
// matrix W (row o - n_q).  Either part may be empty.
struct ProjArgs {
    const float *x;        // [T][ldx]
    float *y;              // [T][ldy]
    const int8_t *Q;       // [n_q][I]
    const int8_t *Qt;      // the same int8 rows tiled (tile_q8), or null: the prefill-sized GEMM reads these
    const float *scale;    // [n_q]
    const float *W;        // [O - n_q][I]
    int64_t ldx, ldy;
    int T, I, O, n_q;
    uint16_t *xb;          // scratch for int8 rows with T > 4 (proj_xb_bytes), or null: x as three bf16 planes [3][T][I], fp32 sums over 64-wide k blocks [T][I/64], k-split partial tiles and arrival counters
    size_t xb_n;           // bytes at xb (launch_proj refuses a shape whose scratch does not fit)
    bool x_split;          // x is already in xb, in the layout the kernel takes (written by the decode core)
    int *counters;         // or null: k-split arrival counters that are zero between launches (each tile's
    int ncounters;         //   last arriver resets its own), so no launch has to clear them
    float *part;           // (set by launch_proj from xb)
    int *cnt;
    // or null: x is a decode core's gated output before its 1 / rms (T <= 4
    // tokens, int8 rows only), which the GEMV applies as it loads x: x_i * rn,
    // rn = (sum of the head's 4 partial sums of squares in slice order / gvd
    // + geps)^-1/2, partial (t, head, slice) at gssq[(t * (I / gvd) + head) * 4 + slice]
    const float *gssq;
    int gvd;
    float geps;
};
// bytes of the scratch a projection of T tokens over I inputs into n_q int8 rows uses
size_t proj_xb_bytes(int T, int I, int n_q);
// whether that projection takes x as int8 planes (i8_off layout) rather than
// bf16 planes (xpiece layout): what a kernel writing x ahead must produce
bool proj_x_int8_planes(int T, int I, int n_q);
// hidden size I and int8 row count n_q the projection kernels take
bool proj_supported(int I, int n_q);
hipError_t launch_proj(const ProjArgs &p, hipStream_t st);
// Tiled copy of int8 weights [O][I] for the prefill-sized GEMM: 16-row x
// 64-k fragments, each a contiguous 1 KiB run in v_mfma_i32_16x16x64_i8
// A-operand order (byte 16 L + j of fragment (o / 16, k / 64) holds row
// 16 (o / 16) + L % 16 at k = 64 (k / 64) + 16 (L / 16) + j), fragments
// k-fastest, rows padded to 16 with zeros.  Wanted for I a multiple of 256.
bool tile_q8_wanted(int O, int I);
__host__ __device__ inline size_t tile_q8_bytes(int O, int I) { return (size_t)(O + 15) / 16 * 16 * I; }
hipError_t tile_q8(const int8_t *Q, int O, int I, int8_t *Qt, hipStream_t st);

// Chunked prefill of T tokens of one sequence (kd == vd == D).
constexpr int kChunk = 64;
struct PrefillArgs {
    // inputs, token-major rows
    const float *qkv; int64_t ld_qkv;    // [T][>= conv_dim]
    const float *z;   int64_t ld_z;      // [T][>= vh*vd]
    const float *a, *b; int64_t ld_ab;   // [T][>= vh]
    float *core;                         // [T][vh*vd]
    // the sequence's state and the layer's weights
    LayerPtrs L;
    int seq;
    int T, Tp, nc;                       // tokens, padded to kChunk, chunks
    int kh, vh, K;
    float eps;
    // scratch (device), sized by prefill_scratch_bytes()
    float *glast;                        // exp(cumulative log-decay at chunk end) [vh][nc]
    float *pg, *pe;                      // e^{gc}, e^{gc_last - gc} per token [vh][nc][C]
    float *pw, *pa, *pu;                 // per (value head, chunk) operand panels (WY kernel -> scan)
    float *pq, *pk;                      // q^, k^ per (key head, chunk), shared by its value heads
};
size_t prefill_scratch_bytes(int D, int kh, int vh, int T);
void prefill_bind_scratch(PrefillArgs &a, int D, void *base);
bool prefill_supported(int kd, int vd, int rep, int K);
hipError_t launch_prefill_core(const PrefillArgs &a, int D, hipStream_t st);

// Copy of one sequence's whole state (S block, conv ring, ring phase of the
// epoch the next launch reads) over another's, for nl layers of one shape.
struct StateCopyArgs {
    const float *S_src[kMaxDecodeLayers], *R_src[kMaxDecodeLayers];
    float *S_dst[kMaxDecodeLayers], *R_dst[kMaxDecodeLayers];
    const int *P_src[kMaxDecodeLayers];
    int *P_dst[kMaxDecodeLayers];
    size_t n4, r4;                     // float4s of S and of the ring per sequence
    int nl;
};
hipError_t launch_state_copy(const StateCopyArgs &c, hipStream_t st);

// Gated full attention (engines/qwen.c:366-425) for T tokens of sequence
// seq at positions pos .. pos+T-1, after the qkv projection.
constexpr int kAttnMaxGroup = 16;     // query heads per kv head
struct AttnArgs {
    const float *qkv; int64_t ld_qkv;  // [T] rows: H x (hd q, hd gate), KV x hd k, KV x hd v
    const float *qn, *kn;              // [hd] RMSNorm weights of q and k (applied as 1 + w)
    const float *inv;                  // [rot / 2] RoPE inverse frequencies
    float *Kc, *Vc;                    // [max_seqs][KV][max_t][hd] caches
    float *qb;                         // [T][H][hd] scratch: q after norm and RoPE
    float *po, *pml;                   // [T][H][ns][hd] partial outputs, [T][H][ns][2] running max and sum
    float *ctx;                        // [T][H * hd] gated attention output
    int seq, pos, T, H, KV, rot, max_t;
    int ns, kps;                       // key splits and keys per split (attn_plan)
    float eps, scale;                  // RMSNorm eps, hd^-1/2
    unsigned char *img;                // or null: the bf16 x 3 flash kernel's tile images [KV][img_tiles][stage]
    int img_tiles;                     //   (attn_flash_image_bytes), made in the same call from the cache
};
bool attn_supported(int hd, int H, int KV, int rot);
// bytes of the tile images a prompt step of T tokens at position pos takes
// (keys 0 .. pos + T - 1 of each kv head; *tiles = tiles per kv head), or 0
// (*tiles = 0) where its flash kernel stages tiles itself
size_t attn_flash_image_bytes(int hd, int KV, int pos, int T, int *tiles);
// whether a prompt step of T tokens runs on the flash kernel (no split partials)
bool attn_uses_flash(int T, int hd);
// splits for pos + T visible keys: ns * KV * T >= 256 workgroups where the keys allow
void attn_plan(int pos, int T, int KV, int &ns, int &kps);
hipError_t launch_attn(const AttnArgs &a, int hd, hipStream_t st);

// Returns hipSuccess, or hipErrorInvalidValue for an unsupported shape.
// variant: 0 = chosen by launch size; kDecodePaired = one workgroup per key
// head streaming its value heads; 1, 2, 4, 8 = one workgroup per column
// slice of a value head, with that many slices.
constexpr int kDecodePaired = -1;
hipError_t launch_decode_core(const DecodeArgs &args, int kd, int vd, int variant, hipStream_t st);
bool decode_core_supported(int kd, int vd, int rep, int K);
// whether a launch with this variant request can also write the out_proj planes (DecodeArgs::xb)
bool decode_planes_supported(int vd, int variant, bool i8);
// sequences per launch for one layer's B sequences: B, or chunks that each fit one round of resident workgroups
int decode_seqs_per_launch(int kd, int vd, int kh, int vh, int nl, int B, int variant);
// column slices per value head for a launch whose gated norm is left to the
// consumer (DecodeArgs::ssq_out), or 0 where the shape has no such form
int decode_deferred_slices(int kd, int vd);

}  // namespace omh
