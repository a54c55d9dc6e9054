/* omh_qwen_main.h — the batched prompt step and the teacher-forced gate for
 * the reference engine (engines/qwen.c), included right before its serve()
 * (qwen.c:566), so both serve() and the validation main() can use them.
 *
 * The reference feeds a prompt token by token through step() (qwen.c:588,
 * 637).  omh_step_batch() runs T tokens through the stack layer by layer,
 * as the engine's gemma path does (gemma.c:483 step_batch): each GDN layer
 * is one chunked omh_gdn_prefill of all T tokens and each attention layer
 * one omh_attn_forward of T tokens; the norms, the MoE and the head stay the
 * engine's own code, per token.  A layer that is not on the GPU (no device,
 * OM_HIP=0, or a fallback) runs its T tokens through the engine's own
 * deltanet_step / attn_step in order, which is the same recurrence.
 *
 *   serve (--serve)           each request's ids (qwen.c:588) are one
 *                             omh_step_batch call, continuing from the
 *                             current position and state (reset:false) or
 *                             from zero (reset:true); OMH_BATCH_PROMPT=0
 *                             keeps the reference's token-by-token loop;
 *   OMH_BATCH_PROMPT=1        the validation main prefills its prompt in
 *                             one omh_step_batch call instead of np step()s
 *                             (off by default, so the reference's own gate
 *                             runs as the reference runs it);
 *   <engine> --tf ref.json    teacher-forced gate: one omh_step_batch over
 *                             full_ids, argmax per position against the
 *                             reference's tf_argmax (transformers' chunked
 *                             path, tools/make_qwen_oracle.py:68-69);
 *                             exit 0 iff every position matches.
 */
#ifndef OMH_QWEN_MAIN_H
#define OMH_QWEN_MAIN_H

static int *read_ints(jval *o, const char *key, int *n);   /* defined by the engine after serve() */

/* T tokens at positions m->pos ..; logits of every position into
 * all_logits [T][vocab] when it is not NULL; returns the last position's
 * logits (malloc'd, as step() does). */
static float *omh_step_batch(Model *m, const int *ids, int T, float *all_logits) {
    Cfg *c = &m->c;
    const int D = c->hidden, val_dim = c->lin_vh * c->lin_vd;
    const int W = val_dim > D ? val_dim : D;             /* deltanet's [val_dim] scratch (qwen.c:505) */
    float *x = falloc((int64_t)T * D), *nrm = falloc((int64_t)T * D), *tmp = falloc((int64_t)T * W);
    for (int t = 0; t < T; t++) memcpy(x + (int64_t)t * D, m->embed + (int64_t)ids[t] * D, D * sizeof(float));
    for (int i = 0; i < c->n_layers; i++) {
        Layer *l = &m->L[i];
        for (int t = 0; t < T; t++) rmsnorm(nrm + (int64_t)t * D, x + (int64_t)t * D, l->in_ln, D, c->eps);
        double tt = now_s();
        int done = 0;
#ifdef OM_HIP
        if (omh_layer_on(m, l, i, T)) {
            /* the GPU writes out[T][D] densely; tmp rows are D apart here */
            done = !omh_injected_failure(i) &&
                   (l->is_full ? omh_attn_forward(i, 0, m->pos, T, nrm, tmp)
                               : omh_gdn_prefill(i, 0, T, nrm, tmp)) == 0;
            if (!done) omh_fallback(m, l->is_full ? "omh_attn_forward (prompt)" : "omh_gdn_prefill", T);
        }
#endif
        if (!done) {
            float *one = falloc(W);
            for (int t = 0; t < T; t++) {
                if (l->is_full) attn_step(m, l, i, nrm + (int64_t)t * D, m->pos + t, one);
                else deltanet_step(m, l, i, nrm + (int64_t)t * D, one);
                memcpy(tmp + (int64_t)t * D, one, D * sizeof(float));
            }
            free(one);
        }
        if (l->is_full) g_t_attn += now_s() - tt; else g_t_delta += now_s() - tt;
        for (int64_t j = 0; j < (int64_t)T * D; j++) x[j] += tmp[j];
        tt = now_s();
        for (int t = 0; t < T; t++) {
            rmsnorm(nrm, x + (int64_t)t * D, l->post_ln, D, c->eps);
            moe_step(m, l, nrm, tmp);
            for (int j = 0; j < D; j++) x[(int64_t)t * D + j] += tmp[j];
        }
        g_t_moe += now_s() - tt;
    }
    m->pos += T;
    float *logit = falloc(c->vocab);
    for (int t = all_logits ? 0 : T - 1; t < T; t++) {
        rmsnorm(nrm, x + (int64_t)t * D, m->final_norm, D, c->eps);
        double tt = now_s();
        if (m->stream) matmul_q(logit, nrm, m->Qlmh.q, m->Qlmh.s, D, c->vocab);
        else matvec(logit, nrm, m->lm_head, D, c->vocab);
        g_t_head += now_s() - tt;
        if (all_logits) memcpy(all_logits + (int64_t)t * c->vocab, logit, c->vocab * sizeof(float));
    }
    free(x); free(nrm); free(tmp);
    return logit;
}

static int omh_batch_prompt(void) {
    const char *e = getenv("OMH_BATCH_PROMPT");
    return e && e[0] == '1';
}

/* Placed in front of the validation main's prompt loop (qwen.c:637): with
 * OMH_BATCH_PROMPT=1 the prompt is one batched step, else the loop runs. */
#define OMH_PROMPT(m, ids, n, logit) \
    if (omh_batch_prompt()) { free(logit); logit = omh_step_batch((m), (ids), (n), NULL); } else

/* serve()'s request ids (a JSON array, PROTOCOL.md) as one batched step. */
static int omh_serve_batch(void) {
    const char *e = getenv("OMH_BATCH_PROMPT");
    return !(e && e[0] == '0');
}
static float *omh_serve_prompt(Model *m, jval *jids, int nids) {
    int *ids = malloc((size_t)nids * sizeof(int));
    for (int i = 0; i < nids; i++) ids[i] = (int)jids->kids[i]->num;
    float *logit = omh_step_batch(m, ids, nids, NULL);
    free(ids);
    return logit;
}

/* Placed in front of serve()'s prompt loop (qwen.c:588). */
#define OMH_SERVE_PROMPT(m, jids, nids, logit) \
    if (omh_serve_batch() && (nids) > 0) { free(logit); logit = omh_serve_prompt((m), (jids), (nids)); } else

/* Teacher-forced gate over ref.json's full_ids against tf_argmax. */
static int omh_tf_gate(const char *snap, const char *refpath) {
    FILE *f = fopen(refpath, "rb");
    if (!f) { perror(refpath); return 1; }
    fseek(f, 0, SEEK_END); long n = ftell(f); fseek(f, 0, SEEK_SET);
    char *buf = malloc(n + 1);
    if (fread(buf, 1, n, f) != (size_t)n) { fclose(f); return 1; }
    buf[n] = 0; fclose(f);
    char *arena = NULL; jval *ref = json_parse(buf, &arena);
    int nf = 0, ntf = 0;
    int *full = read_ints(ref, "full_ids", &nf), *tf = read_ints(ref, "tf_argmax", &ntf);
    if (nf < 1 || ntf != nf) { fprintf(stderr, "tf gate: %s lacks full_ids / tf_argmax\n", refpath); return 1; }
    Model m; memset(&m, 0, sizeof(m));
    model_init(&m, snap, nf + 8);
    float *all = falloc((int64_t)nf * m.c.vocab);
    double t0 = now_s();
    free(omh_step_batch(&m, full, nf, all));
    fprintf(stderr, "teacher-forced: %d positions in one batched step, %.3fs\n", nf, now_s() - t0);
    int match = 0;
    printf("tf_argmax: "); for (int i = 0; i < nf; i++) printf("%d ", tf[i]);
    printf("\nengine   : ");
    for (int i = 0; i < nf; i++) {
        const float *lg = all + (int64_t)i * m.c.vocab;
        int best = 0;
        for (int v = 1; v < m.c.vocab; v++) if (lg[v] > lg[best]) best = v;
        printf("%d ", best);
        match += best == tf[i];
    }
    printf("\nteacher-forced match: %d/%d %s\n", match, nf, match == nf ? "EXACT" : "");
    return match == nf ? 0 : 1;
}

/* First line of the validation main: `--tf ref.json` runs the gate above. */
#define OMH_MAIN_HOOK(argc, argv) \
    do { \
        if ((argc) > 2 && !strcmp((argv)[1], "--tf")) { \
            const char *snap_ = getenv("SNAP"); \
            if (!snap_) { fprintf(stderr, "set SNAP=<model dir>\n"); return 1; } \
            return omh_tf_gate(snap_, (argv)[2]); \
        } \
    } while (0)

#endif
