/* gdn_oracle.h — CPU restatement of the reference Gated DeltaNet (GDN) layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load or call it.  No product code path routes through it.
 *
 * Every function restates the reference engine (overhang engines/qwen.c) with
 * the same operation order, so that, built without FMA contraction, it is
 * bit-identical to the reference's own deltanet_step; tests/test_oracle.py
 * pins that against fixtures written by the compiled reference (oracle/_ref).
 *
 * Layouts (all row-major, fp32 unless stated):
 *   W[O][I] projection weights; conv_w[conv_dim][K]; conv_st[conv_dim][K-1]
 *   (oldest..newest); S[vh][kd][vd]; conv_dim = 2*kh*kd + vh*vd.
 */
#ifndef GDN_ORACLE_H
#define GDN_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int kh, vh, kd, vd;   /* linear_num_key_heads, linear_num_value_heads, key/value head dims */
    int K;                /* linear_conv_kernel_dim */
    int hidden;           /* hidden_size D */
    float eps;            /* rms_norm_eps (gated norm) */
} gdno_dims;

typedef struct {
    /* fp32 projections, row-major [O][I] */
    const float *W_qkv, *W_z, *W_b, *W_a, *W_out;
    /* int8 twins with per-row scales, used when the layer runs in int8 mode
     * (reference "stream" mode: qkv, z, out are int8; b, a stay fp32) */
    const int8_t *Q_qkv, *Q_z, *Q_out;
    const float *S_qkv, *S_z, *S_out;
    const float *conv_w, *A_log, *dt_bias, *gnorm;
} gdno_layer_w;

/* y[O] = W[O][I] x[I], fp32 sequential accumulation (qwen.c:70-77). */
void gdno_matvec(float *y, const float *x, const float *W, int I, int O);
/* per-row absmax int8 quantisation, scale floor 1e-8, lrintf, clamp (qwen.c:124-138). */
void gdno_quantize_rows(const float *w, int8_t *q, float *scale, int O, int I);
/* y[O] = (sum_i x[i]*q[o][i]) * scale[o], x86 scalar branch (qwen.c:116-121). */
void gdno_matmul_q(float *y, const float *x, const int8_t *q, const float *scale, int I, int O);

/* One token of the GDN core for one sequence: causal conv update + SiLU,
 * q/k L2-norm + q scale, gates, delta-rule recurrence, gated RMSNorm
 * (qwen.c:307-358).  qkv[conv_dim] is the in_proj_qkv output, z[vh*vd],
 * a[vh], b[vh]; core[vh*vd] receives the gated-normed head outputs.
 * conv_st and S are updated in place. */
void gdno_core_step(const gdno_dims *d, const float *conv_w, const float *A_log,
                    const float *dt_bias, const float *gnorm,
                    const float *qkv, const float *z, const float *a, const float *b,
                    float *conv_st, float *S, float *core);
/* T tokens of gdno_core_step, token-major inputs/outputs. */
void gdno_core_seq(const gdno_dims *d, const float *conv_w, const float *A_log,
                   const float *dt_bias, const float *gnorm, int T,
                   const float *qkv, const float *z, const float *a, const float *b,
                   float *conv_st, float *S, float *core);
/* One token through the whole GDN layer (qwen.c:301-364): projections (fp32,
 * or int8 twins when int8 != 0), core, out_proj.  x[D] -> out[D]. */
void gdno_layer_step(const gdno_dims *d, const gdno_layer_w *w, int int8,
                     const float *x, float *out, float *conv_st, float *S);
/* T tokens of gdno_layer_step. */
void gdno_layer_seq(const gdno_dims *d, const gdno_layer_w *w, int int8, int T,
                    const float *x, float *out, float *conv_st, float *S);

/* Chunked (WY/UT) restatement of the same recurrence on pre-normalised
 * inputs, following transformers torch_chunk_gated_delta_rule
 * (modeling_qwen3_5_moe.py:250-328).  Inputs per token: q,k [T][kh][kd]
 * already L2-normalised (q also scaled by kd^-1/2), v [T][vh][vd],
 * g [T][vh] (log decay), beta [T][vh].  o [T][vh][vd] receives the
 * un-normalised core output; S is the carried state.  Used to pin the
 * chunk algebra (chunk-size invariance) independently of the GPU. */
void gdno_chunked(int kh, int vh, int kd, int vd, int T, int C,
                  const float *q, const float *k, const float *v,
                  const float *g, const float *beta, float *S, float *o);

/* Number of OpenMP threads the oracle runs with (for baseline reports). */
int gdno_threads(void);

#ifdef __cplusplus
}
#endif
#endif
