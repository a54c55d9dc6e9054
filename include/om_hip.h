/* om_hip.h — C-ABI of the MI355X Gated DeltaNet (GDN) layer.
 *
 * The drop-in for the GDN path of the overhang Qwen3.5/3.6 engine
 * (engines/qwen.c).  The engine stays C and keeps its layer call
 *     static void deltanet_step(Model *m, Layer *l, int li, const float *x, float *out)
 * (engines/qwen.c:301); inside it, under -DOM_HIP, it calls omh_gdn_decode()
 * and falls back to its CPU body on any non-zero return.
 *
 * Conventions follow the engine's existing GPU shim (metal/om_metal.h:9-50):
 *   - C linkage, plain pointers and sizes;
 *   - omh_init() returns 1 = ready, 0 = unavailable, memoised; OM_HIP=0 in
 *     the environment opts out (the OM_METAL=0 precedent, engines/olmoe.c:22-29);
 *   - entry points return 0 on success, a negative OMH_ERR_* code otherwise
 *     (om_metal.mm:168,197,267), and the caller falls back to the CPU;
 *   - host-pointer entry points are synchronous (om_metal's
 *     waitUntilCompleted); the *_dev variants take device pointers and a
 *     hipStream_t (as void*, NULL = the null stream) and only enqueue.
 *
 * Layouts are the reference's, row-major fp32 unless stated:
 *   projection weights W[O][I]; int8 twins q[O][I] + per-row scale s[O]
 *   (engines/qwen.c:34, 124-138); conv1d weight [conv_dim][K]; conv state
 *   [conv_dim][K-1] oldest..newest (qwen.c:275, 308); recurrent state
 *   S[vh][kd][vd] (qwen.c:276, 332); conv_dim = 2*kh*kd + vh*vd;
 *   mixed_qkv = [q | k | v] channels (qwen.c:321).
 *
 * After the first successful GPU call for a layer the device state is the
 * authoritative copy; a caller that falls back to the CPU mid-sequence must
 * first fetch it with omh_gdn_state_get().
 */
#ifndef OM_HIP_H
#define OM_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define OMH_OK            0
#define OMH_ERR_ALLOC    -1   /* device allocation failed                  */
#define OMH_ERR_ARG      -2   /* unknown layer/sequence, bad pointer/size  */
#define OMH_ERR_SHAPE    -3   /* shape not supported by the kernels        */
#define OMH_ERR_DEVICE   -4   /* no usable gfx950 device / HIP error       */

/* 1 = an MI355X (gfx950) is ready, 0 = unavailable.  Memoised.  Replaces
 * omm_init (metal/om_metal.h:13-14) for this path. */
int omh_init(void);

/* Text of the last error on this thread's most recent failing call. */
const char *omh_last_error(void);

/* GDN layer dimensions: the linear_* fields the engine reads from
 * config.json (engines/qwen.c:190-192, 196) plus hidden_size. */
typedef struct {
    int kh, vh, kd, vd;   /* linear_num_key/value_heads, linear_key/value_head_dim */
    int conv_k;           /* linear_conv_kernel_dim                               */
    int hidden;           /* hidden_size (0 for a core-only layer)                */
    float eps;            /* rms_norm_eps, used by the gated norm                 */
} omh_gdn_dims;

/* Host copies of one layer's weights, as the engine's Layer holds them
 * (engines/qwen.c:42, 47).  Projections may be fp32 (W_*) or int8 twins
 * (Q_*, S_*); when a Q_ pointer is non-NULL it is used.  in_proj_b and
 * in_proj_a are always fp32, as in the engine (qwen.c:324-325).  All
 * projection pointers may be NULL for a core-only layer. */
typedef struct {
    const float *W_qkv, *W_z, *W_b, *W_a, *W_out;
    const int8_t *Q_qkv, *Q_z, *Q_out;
    const float *S_qkv, *S_z, *S_out;
    const float *conv_w;             /* [conv_dim][K] */
    const float *A_log, *dt_bias;    /* [vh]          */
    const float *gnorm;              /* [vd]          */
} omh_gdn_weights;

/* Upload a layer's weights (copied; the host keeps its arrays) and allocate
 * zeroed conv + recurrent state for max_seqs sequences.  Replaces the
 * per-layer state allocation of model_init (engines/qwen.c:259-276).
 * li in [0, 4096).  Re-initialising an existing li replaces it. */
int omh_gdn_layer_init(int li, const omh_gdn_dims *d, const omh_gdn_weights *w, int max_seqs);
int omh_gdn_layer_free(int li);

/* Zero one sequence's conv and recurrent state (seq < 0: every sequence):
 * the reset branch of serve() (engines/qwen.c:576-582). */
int omh_gdn_state_reset(int li, int seq);
/* Copy one sequence's state out / in, in the reference layouts
 * (conv [conv_dim][K-1], S [vh][kd][vd]); either pointer may be NULL. */
int omh_gdn_state_get(int li, int seq, float *conv, float *S);
int omh_gdn_state_set(int li, int seq, const float *conv, const float *S);

/* ---- host-pointer, synchronous entry points (the engine's drop-in) ---- */

/* One token for each of sequences 0..B-1 through the whole layer:
 * x[B][hidden] (the input-layernorm output) -> out[B][hidden] (the out_proj
 * output the caller adds to its residual).  B = 1 is exactly
 * deltanet_step(m, l, li, x, out) (engines/qwen.c:301-364). */
int omh_gdn_decode(int li, int B, const float *x, float *out);

/* T consecutive tokens of sequence seq through the whole layer, continuing
 * from its current state (chunked WY/UT form on the GPU).  Equivalent to T
 * calls of deltanet_step; x[T][hidden] -> out[T][hidden].  New capability:
 * the engine prefills token by token (engines/qwen.c:588, 637). */
int omh_gdn_prefill(int li, int seq, int T, const float *x, float *out);

/* Device-side snapshot / rollback for speculative decoding: for each of
 * the nl layers lis[] (all of one shape), copy sequence src_seq's whole GDN
 * state (recurrent state, conv history and its ring position) over sequence
 * dst_seq's, device to device, in one launch.  Snapshot = copy into a spare
 * sequence slot before the speculative tokens; rollback = copy it back after
 * a rejection.  The reference has no counterpart: its worklog records
 * rollback as infeasible for the deltanet state as implemented
 * (WORKLOG.md:157-158), and multi-token prediction is on its roadmap
 * (ROADMAP.md:10).  The _dev variant enqueues on `stream`. */
int omh_gdn_state_copy(int nl, const int *lis, int src_seq, int dst_seq);
int omh_gdn_state_copy_dev(int nl, const int *lis, int src_seq, int dst_seq, void *stream);

/* Core only (no projections): pre-projected mixed_qkv[B][conv_dim],
 * z[B][vh*vd], a[B][vh], b[B][vh] -> core[B][vh*vd], the gated-normed head
 * outputs that out_proj consumes (engines/qwen.c:307-358). */
int omh_gdn_decode_core(int li, int B, const float *qkv, const float *z,
                        const float *a, const float *b, float *core);
/* Core only, T tokens of one sequence: inputs/outputs [T][...]. */
int omh_gdn_prefill_core(int li, int seq, int T, const float *qkv, const float *z,
                         const float *a, const float *b, float *core);

/* ---- device-pointer, stream-ordered variants (asynchronous) ----
 *
 * They share the library's scratch and each layer's state with every other
 * entry point: calls that may overlap in time must be issued on one stream.
 * The host-pointer calls above run on a stream of the library's own and do
 * not wait for work a caller enqueued on its streams; call omh_sync() on
 * those streams first. */

/* Core decode for nl layers at once (nl >= 1, all of identical dims), each
 * with B sequences: inputs [nl][B][...] and core [nl][B][vh*vd] in device
 * memory; lis[nl] is a host array of layer ids.  Layers are independent
 * here (pre-projected inputs), so one launch serves them all. */
int omh_gdn_decode_core_dev(int nl, const int *lis, int B, const float *qkv, const float *z,
                            const float *a, const float *b, float *core, void *stream);
/* The same for sequences seq0 .. seq0+B-1 of every listed layer (a server
 * stepping some of its sequence slots); inputs and core are [nl][B][...]
 * as above.  omh_gdn_decode_core_dev is seq0 = 0.  No counterpart in the
 * reference, which runs one sequence (engines/qwen.c:566-607). */
int omh_gdn_decode_core_seq_dev(int nl, const int *lis, int seq0, int B, const float *qkv, const float *z,
                                const float *a, const float *b, float *core, void *stream);
int omh_gdn_prefill_core_dev(int li, int seq, int T, const float *qkv, const float *z,
                             const float *a, const float *b, float *core, void *stream);
int omh_gdn_decode_dev(int li, int B, const float *x, float *out, void *stream);
int omh_gdn_prefill_dev(int li, int seq, int T, const float *x, float *out, void *stream);

/* omh_gdn_decode_dev without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory mid-run: code
 * under HIP graph capture, fixed-footprint serving loops, harnesses that
 * forbid hipMalloc.  Same computation and kernels as omh_gdn_decode_dev, but
 * its scratch (in_proj rows, core rows, the core slices' sums of squares,
 * the int8 projections' x planes, partial tiles and arrival counters) is one
 * static 8 MiB device buffer per GPU, held until the process ends, instead
 * of the library's grow-only scratch.  A call whose scratch would exceed 8 MiB returns OMH_ERR_SHAPE
 * (35B-A3B GDN shape: up to B = 64 fits).  All calls on one GPU share that
 * buffer, so calls that may overlap in time (different streams) race:
 * issue them from one stream. */
int omh_gdn_decode_noalloc_dev(int li, int B, const float *x, float *out, void *stream);

/* Wait for all work this library enqueued on `stream`. */
int omh_sync(void *stream);

/* ---- gated full-attention layer (the 1-in-4 non-GDN layer) ---- */

/* Dimensions as the engine reads them from config.json: num_attention_heads,
 * num_key_value_heads, head_dim, rot_dim = head_dim * partial_rotary_factor,
 * rope_theta, rms_norm_eps (engines/qwen.c:367-369), plus the KV cache
 * length max_t (the engine's m->max_t, qwen.c:257-258). */
typedef struct {
    int hidden;
    int n_heads, n_kv, head_dim, rot_dim;
    float theta, eps;
    int max_t;
} omh_attn_dims;

/* The layer's tensors (engines/qwen.c:244-255): q_proj [2*H*hd][hidden]
 * (per head [hd q | hd gate], qwen.c:376-382), k_proj and v_proj
 * [KV*hd][hidden], o_proj [hidden][H*hd], each fp32 or int8 + per-row
 * scale (all three of q/k/v in one form); q_norm, k_norm [hd]. */
typedef struct {
    const float *W_q, *W_k, *W_v, *W_o;
    const int8_t *Q_q, *Q_k, *Q_v, *Q_o;
    const float *S_q, *S_k, *S_v, *S_o;
    const float *q_norm, *k_norm;
} omh_attn_weights;

/* Attention layer ids are a namespace of their own, separate from the GDN
 * layer ids.  The K and V caches ([max_seqs][n_kv][max_t][head_dim] each,
 * the engine's m->K[li] / m->V[li] per sequence) live on the device. */
int omh_attn_layer_init(int li, const omh_attn_dims *d, const omh_attn_weights *w, int max_seqs);
int omh_attn_layer_free(int li);

/* T tokens x[T][hidden] of sequence seq at positions pos .. pos+T-1 ->
 * out[T][hidden]; writes their K and V into the cache and attends causally
 * over positions 0 .. pos+t, which earlier calls must have written.  T = 1
 * replaces attn_step(m, l, li, x, pos, out) (engines/qwen.c:367); T > 1 is
 * the batched prompt step the engine runs token by token
 * (qwen.c:588, 637).  Requires pos + T <= max_t. */
int omh_attn_forward(int li, int seq, int pos, int T, const float *x, float *out);
int omh_attn_forward_dev(int li, int seq, int pos, int T, const float *x, float *out, void *stream);

/* Copy cache rows t0 .. t0+n-1 of every kv head of sequence seq out of /
 * into the device, from host arrays in the engine's layout
 * [n_kv][ld_t][head_dim] (m->K[li] / m->V[li] with ld_t = m->max_t,
 * engines/qwen.c:257-258; rows written at qwen.c:399-402).  Either pointer
 * may be NULL.  After the first successful omh_attn_forward the device
 * cache is the authoritative copy: a caller that falls back to the CPU
 * mid-sequence first fetches rows 0 .. pos with omh_attn_cache_get (the
 * counterpart of omh_gdn_state_get); cache_set re-seeds a layer that moves
 * to the GPU mid-sequence.  Synchronous. */
int omh_attn_cache_get(int li, int seq, int t0, int n, float *K, float *V, int ld_t);
int omh_attn_cache_set(int li, int seq, int t0, int n, const float *K, const float *V, int ld_t);

#ifdef __cplusplus
}
#endif
#endif
