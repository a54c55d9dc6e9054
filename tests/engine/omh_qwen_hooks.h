/* omh_qwen_hooks.h — the OM_HIP hooks of the reference engine's GDN and
 * gated-attention layers (engines/qwen.c), as a maintainer would add them.
 *
 * tests/engine/Makefile compiles the reference engines/qwen.c with this file
 * included right before deltanet_step (so Model, Layer, Cfg and the engine's
 * helpers are in scope) and one hook line at the top of deltanet_step
 * (qwen.c:301) and attn_step (qwen.c:367).  Without -DOM_HIP the hooks are
 * empty and the engine is the reference's.
 *
 * Conventions are the engine's existing GPU shim's (om_metal, engines/olmoe.c
 * :22-29, 289, 379-382): omh_init() once, OM_HIP=0 opts out, any non-zero
 * return falls back to the CPU body.  Layers are uploaded on first use (the
 * om_metal weight cache keyed by host pointer, metal/om_metal.mm:250-261,
 * likewise fills itself on first use), so model_init is unchanged.  On a
 * fallback every layer already on the GPU hands its state back first: the
 * GDN conv/recurrent state (omh_gdn_state_get) and the attention cache rows
 * (omh_attn_cache_get), because after the first GPU call the device copy is
 * the authoritative one.
 */
#ifndef OMH_QWEN_HOOKS_H
#define OMH_QWEN_HOOKS_H

#ifdef OM_HIP
#include "om_hip.h"

static int omh_on = -1;                  /* -1: not asked yet; 1: GPU; 0: CPU */
static unsigned char *omh_up;            /* per engine layer: 1 = on the device */
static int omh_nl;

static int omh_ready(Model *m) {
    if (omh_on < 0) {
        omh_on = omh_init();
        omh_nl = m->c.n_layers;
        omh_up = calloc(omh_nl > 0 ? omh_nl : 1, 1);
        if (!omh_up) omh_on = 0;
        fprintf(stderr, omh_on == 1 ? "om_hip: GDN and attention layers on the GPU (gfx950)\n"
                                    : "om_hip: GPU path off (%s); CPU layers\n", omh_last_error());
    }
    return omh_on == 1;
}

/* Test-only fault injection, from the host (no GPU call is made for it):
 * OMH_TEST_FAIL_LAYER=k makes the GPU call of engine layer k report a
 * failure, so the fallback below runs mid-step.  Unset: never. */
static int omh_fail_layer = -2;          /* -2: not read yet; -1: off */
static int omh_injected = 0;             /* the last failure was injected */
static int omh_injected_failure(int li) {
    if (omh_fail_layer == -2) {
        const char *e = getenv("OMH_TEST_FAIL_LAYER");
        omh_fail_layer = e && e[0] ? atoi(e) : -1;
    }
    omh_injected = li == omh_fail_layer;
    return omh_injected;
}

/* Hand every uploaded layer's state back to the engine's arrays and stay on
 * the CPU from here on.  nt: tokens of the step in progress (1 for step(),
 * T for a batched prompt step), so attention layers that ran earlier in it
 * have written cache rows up to pos + nt - 1 on the device: all of rows
 * 0 .. pos + nt - 1 come back (the failing layer's own rows are rewritten by
 * its CPU body next). */
static void omh_fallback(Model *m, const char *where, int nt) {
    fprintf(stderr, "om_hip: %s failed (%s); continuing on the CPU\n", where,
            omh_injected ? "injected by OMH_TEST_FAIL_LAYER" : omh_last_error());
    const long want = (long)m->pos + (nt > 0 ? nt : 1);
    int rows = want < m->max_t ? (int)want : m->max_t;
    for (int i = 0; i < omh_nl; i++) {
        if (!omh_up[i]) continue;
        if (m->L[i].is_full) omh_attn_cache_get(i, 0, 0, rows, m->K[i], m->V[i], m->max_t);
        else omh_gdn_state_get(i, 0, m->conv_st[i], m->rec_st[i]);
    }
    omh_on = 0;
}

static int omh_gdn_upload(Model *m, Layer *l, int li) {
    Cfg *c = &m->c;
    omh_gdn_dims d = {c->lin_kh, c->lin_vh, c->lin_kd, c->lin_vd, c->conv_k, c->hidden, c->eps};
    omh_gdn_weights w;
    memset(&w, 0, sizeof(w));
    w.W_b = l->b; w.W_a = l->a;                       /* fp32 in both modes (qwen.c:324-325) */
    w.conv_w = l->conv_w; w.A_log = l->A_log; w.dt_bias = l->dt_bias; w.gnorm = l->gnorm;
    if (m->stream) {                                  /* int8 twins made at load (qwen.c:269-274) */
        w.Q_qkv = l->Qqkv.q; w.S_qkv = l->Qqkv.s;
        w.Q_z = l->Qz.q;     w.S_z = l->Qz.s;
        w.Q_out = l->Qout.q; w.S_out = l->Qout.s;
    } else {
        w.W_qkv = l->qkv; w.W_z = l->z; w.W_out = l->outp;
    }
    if (omh_gdn_layer_init(li, &d, &w, 1) != 0) return -1;
    /* continue from the engine's current state (zero at the start) */
    return omh_gdn_state_set(li, 0, m->conv_st[li], m->rec_st[li]) == 0 ? 0 : -1;
}

static int omh_attn_upload(Model *m, Layer *l, int li) {
    Cfg *c = &m->c;
    omh_attn_dims d = {c->hidden, c->n_heads, c->n_kv, c->head_dim, c->rot_dim, c->theta, c->eps, m->max_t};
    omh_attn_weights w;
    memset(&w, 0, sizeof(w));
    w.q_norm = l->qn; w.k_norm = l->kn;
    if (m->stream) {                                  /* int8 twins (qwen.c:252-255) */
        w.Q_q = l->Qq.q; w.S_q = l->Qq.s; w.Q_k = l->Qk.q; w.S_k = l->Qk.s;
        w.Q_v = l->Qv.q; w.S_v = l->Qv.s; w.Q_o = l->Qo.q; w.S_o = l->Qo.s;
    } else {
        w.W_q = l->q; w.W_k = l->k; w.W_v = l->v; w.W_o = l->o;
    }
    if (omh_attn_layer_init(li, &d, &w, 1) != 0) return -1;
    /* a layer that moves to the GPU mid-sequence takes the rows written so far */
    return omh_attn_cache_set(li, 0, 0, m->pos, m->K[li], m->V[li], m->max_t) == 0 ? 0 : -1;
}

/* Whether layer li runs on the GPU; uploads it on first use.  nt: tokens of
 * the step in progress (see omh_fallback). */
static int omh_layer_on(Model *m, Layer *l, int li, int nt) {
    if (!omh_ready(m) || li < 0 || li >= omh_nl) return 0;
    if (!omh_up[li]) {
        if ((l->is_full ? omh_attn_upload(m, l, li) : omh_gdn_upload(m, l, li)) != 0) {
            omh_fallback(m, l->is_full ? "attention layer upload" : "GDN layer upload", nt);
            return 0;
        }
        omh_up[li] = 1;
    }
    return 1;
}

/* deltanet_step's hook: 1 = done on the GPU. */
static int omh_gdn_hook(Model *m, Layer *l, int li, const float *x, float *out) {
    if (!omh_layer_on(m, l, li, 1)) return 0;
    if (!omh_injected_failure(li) && omh_gdn_decode(li, 1, x, out) == 0) return 1;
    omh_fallback(m, "omh_gdn_decode", 1);
    return 0;
}

/* attn_step's hook: 1 = done on the GPU. */
static int omh_attn_hook(Model *m, Layer *l, int li, const float *x, int pos, float *out) {
    if (!omh_layer_on(m, l, li, 1)) return 0;
    if (!omh_injected_failure(li) && omh_attn_forward(li, 0, pos, 1, x, out) == 0) return 1;
    omh_fallback(m, "omh_attn_forward", 1);
    return 0;
}

/* serve()'s reset branch (qwen.c:576-582): zero the device GDN states too;
 * the attention caches need nothing (positions restart at 0). */
static void omh_reset(Model *m) {
    if (omh_on != 1) return;
    for (int i = 0; i < omh_nl; i++)
        if (omh_up[i] && !m->L[i].is_full && omh_gdn_state_reset(i, 0) != 0) {
            omh_fallback(m, "omh_gdn_state_reset", 1);
            return;
        }
}

#define OMH_GDN_HOOK(m, l, li, x, out) \
    do { if (omh_gdn_hook((m), (l), (li), (x), (out))) return; } while (0)
#define OMH_ATTN_HOOK(m, l, li, x, pos, out) \
    do { if (omh_attn_hook((m), (l), (li), (x), (pos), (out))) return; } while (0)
#define OMH_RESET(m) omh_reset(m)

#else  /* !OM_HIP: the reference engine unchanged */

#define OMH_GDN_HOOK(m, l, li, x, out) do { } while (0)
#define OMH_ATTN_HOOK(m, l, li, x, pos, out) do { } while (0)
#define OMH_RESET(m) do { } while (0)

#endif
#endif
