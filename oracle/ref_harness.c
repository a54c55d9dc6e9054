/* ref_harness.c — builds the reference engine's own GDN code into a checker.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile, from the reference
 * sources where they lie (REF=/root/reference), into oracle/_ref/ — never
 * committed, never part of the product.  tests/golden/make_golden.py calls
 * it to write golden vectors, and tests/test_oracle.py uses it (when built)
 * to check the restatement in gdn_oracle.c bit for bit.
 *
 * The reference keeps deltanet_step and its helpers `static` inside
 * engines/qwen.c; including the file here gives this translation unit access
 * to them.  Its main() is renamed so it does not clash.
 */
#define main qwen_reference_main
#include "qwen.c"
#undef main

/* One GDN layer run token by token through the reference deltanet_step
 * (qwen.c:301-364) on a synthetic Model/Layer.  stream != 0 quantises
 * qkv/z/out with the reference's qw_make (qwen.c:142-147) first, which is
 * the int8 path of DM (qwen.c:139-141).  conv_st/rec_st are in/out. */
int ref_gdn_layer_run(int kh, int vh, int kd, int vd, int K, int hidden, float eps, int stream,
                      const float *W_qkv, const float *W_z, const float *W_b, const float *W_a,
                      const float *W_out, const float *conv_w, const float *A_log,
                      const float *dt_bias, const float *gnorm,
                      int T, const float *x, float *out, float *conv_st, float *rec_st) {
    Model m; memset(&m, 0, sizeof(m));
    Layer l; memset(&l, 0, sizeof(l));
    m.c.hidden = hidden; m.c.lin_kh = kh; m.c.lin_vh = vh; m.c.lin_kd = kd; m.c.lin_vd = vd;
    m.c.conv_k = K; m.c.eps = eps;
    m.stream = stream;
    const int key_dim = kh * kd, val_dim = vh * vd, conv_dim = 2 * key_dim + val_dim;
    float *cp[5]; const float *src[5] = {W_qkv, W_z, W_b, W_a, W_out};
    const int64_t nel[5] = {(int64_t)conv_dim * hidden, (int64_t)val_dim * hidden,
                            (int64_t)vh * hidden, (int64_t)vh * hidden, (int64_t)hidden * val_dim};
    for (int i = 0; i < 5; i++) {
        cp[i] = falloc(nel[i]);
        memcpy(cp[i], src[i], nel[i] * sizeof(float));
    }
    l.qkv = cp[0]; l.z = cp[1]; l.b = cp[2]; l.a = cp[3]; l.outp = cp[4];
    l.conv_w = (float *)conv_w; l.A_log = (float *)A_log; l.dt_bias = (float *)dt_bias;
    l.gnorm = (float *)gnorm;
    if (stream) {
        l.Qqkv = qw_make(&l.qkv, conv_dim, hidden);
        l.Qz = qw_make(&l.z, val_dim, hidden);
        l.Qout = qw_make(&l.outp, hidden, val_dim);
    }
    float *convs[1] = {conv_st}, *recs[1] = {rec_st};
    m.conv_st = convs; m.rec_st = recs;
    float *tmp = falloc(val_dim > hidden ? val_dim : hidden);
    for (int t = 0; t < T; t++) {
        deltanet_step(&m, &l, 0, x + (int64_t)t * hidden, tmp);
        memcpy(out + (int64_t)t * hidden, tmp, hidden * sizeof(float));
    }
    free(tmp);
    /* qw_make freed (and NULLed) the fp32 originals it quantised */
    free(l.qkv); free(l.z); free(l.b); free(l.a); free(l.outp);
    if (stream) {
        free(l.Qqkv.q); free(l.Qqkv.s); free(l.Qz.q); free(l.Qz.s); free(l.Qout.q); free(l.Qout.s);
    }
    return 0;
}

/* qwen.c:124-138 */
void ref_quantize_rows(const float *w, int8_t *q, float *scale, int O, int I) {
    quantize_rows(w, q, scale, O, I);
}

/* qwen.c:94-122 (x86 scalar branch) */
void ref_matmul_q(float *y, const float *x, const int8_t *q, const float *scale, int I, int O) {
    matmul_q(y, x, q, scale, I, O);
}

/* qwen.c:70-77 */
void ref_matvec(float *y, const float *x, const float *W, int I, int O) {
    matvec(y, x, W, I, O);
}

/* T tokens through the reference attn_step (qwen.c:367-425) on a synthetic
 * Model/Layer, at positions pos0 .. pos0+T-1 of one sequence.  The cache
 * rows 0 .. pos0-1 are first filled from Kpre / Vpre ([pos0][KV][hd], keys
 * as the cache holds them: normed and rotated), so the step attends over
 * thousands of positions without running the prompt through the layer.
 * stream != 0 quantises q/k/v/o with the reference's qw_make first
 * (qwen.c:252-255), the int8 path of DM.  Knew / Vnew (may be NULL) receive
 * the T cache rows the calls wrote, [T][KV][hd].  attn_step keeps its
 * scores in a float[8192] (qwen.c:407), so pos0 + T <= 8192. */
int ref_attn_run(int hidden, int H, int KV, int hd, int rot, float theta, float eps, int stream,
                 const float *Wq, const float *Wk, const float *Wv, const float *Wo,
                 const float *qn, const float *kn, int pos0, const float *Kpre, const float *Vpre,
                 int T, const float *x, float *out, float *Knew, float *Vnew) {
    if (pos0 < 0 || T < 1 || pos0 + T > 8192) return -2;
    Model m; memset(&m, 0, sizeof(m));
    Layer l; memset(&l, 0, sizeof(l));
    m.c.hidden = hidden; m.c.n_heads = H; m.c.n_kv = KV; m.c.head_dim = hd; m.c.rot_dim = rot;
    m.c.theta = theta; m.c.eps = eps;
    m.stream = stream;
    const int max_t = pos0 + T;
    m.max_t = max_t;
    float *cp[4]; const float *src[4] = {Wq, Wk, Wv, Wo};
    const int64_t nel[4] = {(int64_t)2 * H * hd * hidden, (int64_t)KV * hd * hidden,
                            (int64_t)KV * hd * hidden, (int64_t)hidden * H * hd};
    for (int i = 0; i < 4; i++) {
        cp[i] = falloc(nel[i]);
        memcpy(cp[i], src[i], nel[i] * sizeof(float));
    }
    l.q = cp[0]; l.k = cp[1]; l.v = cp[2]; l.o = cp[3];
    l.qn = (float *)qn; l.kn = (float *)kn;
    if (stream) {
        l.Qq = qw_make(&l.q, 2 * H * hd, hidden);
        l.Qk = qw_make(&l.k, KV * hd, hidden);
        l.Qv = qw_make(&l.v, KV * hd, hidden);
        l.Qo = qw_make(&l.o, hidden, H * hd);
    }
    float *Kc = falloc((int64_t)KV * max_t * hd), *Vc = falloc((int64_t)KV * max_t * hd);
    for (int t = 0; t < pos0; t++)
        for (int h = 0; h < KV; h++) {
            memcpy(Kc + ((int64_t)h * max_t + t) * hd, Kpre + ((int64_t)t * KV + h) * hd, hd * sizeof(float));
            memcpy(Vc + ((int64_t)h * max_t + t) * hd, Vpre + ((int64_t)t * KV + h) * hd, hd * sizeof(float));
        }
    float *Ks[1] = {Kc}, *Vs[1] = {Vc};
    m.K = Ks; m.V = Vs;
    for (int t = 0; t < T; t++)
        attn_step(&m, &l, 0, x + (int64_t)t * hidden, pos0 + t, out + (int64_t)t * hidden);
    for (int t = 0; t < T; t++)
        for (int h = 0; h < KV; h++) {
            if (Knew) memcpy(Knew + ((int64_t)t * KV + h) * hd, Kc + ((int64_t)h * max_t + pos0 + t) * hd, hd * sizeof(float));
            if (Vnew) memcpy(Vnew + ((int64_t)t * KV + h) * hd, Vc + ((int64_t)h * max_t + pos0 + t) * hd, hd * sizeof(float));
        }
    free(Kc); free(Vc);
    free(l.q); free(l.k); free(l.v); free(l.o);
    if (stream) {
        free(l.Qq.q); free(l.Qq.s); free(l.Qk.q); free(l.Qk.s);
        free(l.Qv.q); free(l.Qv.s); free(l.Qo.q); free(l.Qo.s);
    }
    return 0;
}

/* One persistent GDN layer for timing the reference's deltanet_step as the
 * engine runs it: ref_layer_open sets up a synthetic Model/Layer (and, for
 * stream != 0, its int8 twins via qw_make, qwen.c:269-274) once,
 * ref_layer_steps runs T tokens through deltanet_step (one call each,
 * carrying the state), ref_layer_close frees it.  One layer at a time. */
static Model g_rm;
static Layer g_rl;
static float *g_rconv, *g_rrec, *g_rtmp;
static int g_ropen;

void ref_layer_close(void) {
    if (!g_ropen) return;
    free(g_rl.qkv); free(g_rl.z); free(g_rl.b); free(g_rl.a); free(g_rl.outp);
    if (g_rm.stream) {
        free(g_rl.Qqkv.q); free(g_rl.Qqkv.s); free(g_rl.Qz.q); free(g_rl.Qz.s);
        free(g_rl.Qout.q); free(g_rl.Qout.s);
    }
    free(g_rconv); free(g_rrec); free(g_rtmp);
    free(g_rm.conv_st); free(g_rm.rec_st);
    g_ropen = 0;
}

int ref_layer_open(int kh, int vh, int kd, int vd, int K, int hidden, float eps, int stream,
                   const float *W_qkv, const float *W_z, const float *W_b, const float *W_a,
                   const float *W_out, const float *conv_w, const float *A_log,
                   const float *dt_bias, const float *gnorm) {
    ref_layer_close();
    memset(&g_rm, 0, sizeof(g_rm));
    memset(&g_rl, 0, sizeof(g_rl));
    g_rm.c.hidden = hidden; g_rm.c.lin_kh = kh; g_rm.c.lin_vh = vh; g_rm.c.lin_kd = kd; g_rm.c.lin_vd = vd;
    g_rm.c.conv_k = K; g_rm.c.eps = eps;
    g_rm.stream = stream;
    const int key_dim = kh * kd, val_dim = vh * vd, conv_dim = 2 * key_dim + val_dim;
    float **dst[5] = {&g_rl.qkv, &g_rl.z, &g_rl.b, &g_rl.a, &g_rl.outp};
    const float *src[5] = {W_qkv, W_z, W_b, W_a, W_out};
    const int64_t nel[5] = {(int64_t)conv_dim * hidden, (int64_t)val_dim * hidden,
                            (int64_t)vh * hidden, (int64_t)vh * hidden, (int64_t)hidden * val_dim};
    for (int i = 0; i < 5; i++) {
        *dst[i] = falloc(nel[i]);
        memcpy(*dst[i], src[i], nel[i] * sizeof(float));
    }
    g_rl.conv_w = (float *)conv_w; g_rl.A_log = (float *)A_log; g_rl.dt_bias = (float *)dt_bias;
    g_rl.gnorm = (float *)gnorm;
    if (stream) {
        g_rl.Qqkv = qw_make(&g_rl.qkv, conv_dim, hidden);
        g_rl.Qz = qw_make(&g_rl.z, val_dim, hidden);
        g_rl.Qout = qw_make(&g_rl.outp, hidden, val_dim);
    }
    g_rconv = falloc((int64_t)conv_dim * (K - 1));
    g_rrec = falloc((int64_t)vh * kd * vd);
    g_rtmp = falloc(val_dim > hidden ? val_dim : hidden);
    g_rm.conv_st = malloc(sizeof(float *));
    g_rm.rec_st = malloc(sizeof(float *));
    g_rm.conv_st[0] = g_rconv;
    g_rm.rec_st[0] = g_rrec;
    g_ropen = 1;
    return 0;
}

int ref_layer_steps(int T, const float *x, float *out) {
    if (!g_ropen) return -2;
    const int D = g_rm.c.hidden;
    for (int t = 0; t < T; t++) {
        deltanet_step(&g_rm, &g_rl, 0, x + (int64_t)t * D, g_rtmp);
        if (out) memcpy(out + (int64_t)t * D, g_rtmp, D * sizeof(float));
    }
    return 0;
}
