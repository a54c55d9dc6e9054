/* gdn_oracle.c — CPU restatement of the reference GDN layer (test checker only).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py.  See gdn_oracle.h for layouts.
 *
 * Each function follows the cited lines of overhang engines/qwen.c with the
 * same loop nest and the same floating-point operation order, and the same
 * OpenMP decomposition (rows of a projection, conv channels, value heads).
 * Built with -O3 -fopenmp and no FMA contraction it is bit-identical to the
 * reference; tests/test_oracle.py checks that against fixtures produced by
 * the reference code itself.
 */
#include "gdn_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float *oalloc(int64_t n) {
    float *p = (float *)calloc((size_t)(n > 0 ? n : 1), sizeof(float));
    if (!p) { fprintf(stderr, "gdn_oracle: OOM %lld\n", (long long)n); abort(); }
    return p;
}

/* qwen.c:158-160 */
static float o_sigmoid(float z) { return 1.f / (1.f + expf(-z)); }
static float o_silu(float z) { return z * o_sigmoid(z); }
static float o_softplus(float z) { return z > 20.f ? z : log1pf(expf(z)); }

/* qwen.c:153-157: Σx² in double, r = 1/sqrtf(Σ + 1e-6f) */
static void o_l2norm(float *x, int n) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    float r = 1.f / sqrtf((float)ss + 1e-6f);
    for (int i = 0; i < n; i++) x[i] *= r;
}

int gdno_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* qwen.c:70-77 */
void gdno_matvec(float *y, const float *x, const float *W, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        float acc = 0.f;
        for (int i = 0; i < I; i++) acc += x[i] * w[i];
        y[o] = acc;
    }
}

/* qwen.c:124-138 */
void gdno_quantize_rows(const float *w, int8_t *q, float *scale, int O, int I) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        float am = 0.f;
        for (int i = 0; i < I; i++) { float a = fabsf(wr[i]); if (a > am) am = a; }
        float s = am / 127.f;
        if (s < 1e-8f) s = 1e-8f;
        scale[o] = s;
        int8_t *qr = q + (int64_t)o * I;
        for (int i = 0; i < I; i++) {
            int v = (int)lrintf(wr[i] / s);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            qr[i] = (int8_t)v;
        }
    }
}

/* qwen.c:116-121 (the branch x86 builds take: __ARM_NEON undefined) */
void gdno_matmul_q(float *y, const float *x, const int8_t *q, const float *scale, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const int8_t *w = q + (int64_t)o * I;
        float acc = 0.f;
        for (int i = 0; i < I; i++) acc += x[i] * (float)w[i];
        y[o] = acc * scale[o];
    }
}

/* Core of deltanet_step after the input projections: qwen.c:307-358. */
void gdno_core_step(const gdno_dims *d, const float *conv_w, const float *A_log,
                    const float *dt_bias, const float *gnorm,
                    const float *qkv, const float *z, const float *aa, const float *bb,
                    float *conv_st, float *S, float *core) {
    const int kh = d->kh, vh = d->vh, kd = d->kd, vd = d->vd, K = d->K;
    const int key_dim = kh * kd, conv_dim = 2 * key_dim + vh * vd;
    float *cv = oalloc(conv_dim);
    /* causal conv1d update + SiLU: qwen.c:307-320 */
    #pragma omp parallel for schedule(static)
    for (int ch = 0; ch < conv_dim; ch++) {
        const float *w = conv_w + (int64_t)ch * K;
        float *h = conv_st + (int64_t)ch * (K - 1);
        float acc = 0.f;
        for (int j = 0; j < K - 1; j++) acc += w[j] * h[j];
        acc += w[K - 1] * qkv[ch];
        for (int j = 0; j < K - 2; j++) h[j] = h[j + 1];
        h[K - 2] = qkv[ch];
        cv[ch] = o_silu(acc);
    }
    float *q = cv, *k = cv + key_dim, *v = cv + 2 * key_dim;
    /* per-head L2 norm + q scale: qwen.c:326-329 */
    for (int h = 0; h < kh; h++) { o_l2norm(q + h * kd, kd); o_l2norm(k + h * kd, kd); }
    float scale = 1.f / sqrtf((float)kd);
    for (int i = 0; i < key_dim; i++) q[i] *= scale;
    /* per v-head recurrence, k/q head = h / (vh/kh): qwen.c:330-358 */
    const int rep = vh / kh;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < vh; h++) {
        const float *qh = q + (h / rep) * kd, *kt = k + (h / rep) * kd;
        const float *vt = v + h * vd;
        float g = -expf(A_log[h]) * o_softplus(aa[h] + dt_bias[h]);
        float ge = expf(g), beta = o_sigmoid(bb[h]);
        float *Sh = S + (int64_t)h * kd * vd;
        float kv[512], delta[512];                         /* vd <= 512, as qwen.c:340 */
        for (int j = 0; j < vd; j++) kv[j] = 0.f;
        for (int i = 0; i < kd; i++) {
            float *Si = Sh + (int64_t)i * vd;
            float ki = kt[i];
            for (int j = 0; j < vd; j++) { Si[j] *= ge; kv[j] += Si[j] * ki; }
        }
        for (int j = 0; j < vd; j++) delta[j] = (vt[j] - kv[j]) * beta;
        float *oh = core + h * vd;
        for (int j = 0; j < vd; j++) oh[j] = 0.f;
        for (int i = 0; i < kd; i++) {
            float *Si = Sh + (int64_t)i * vd;
            float ki = kt[i], qi = qh[i];
            for (int j = 0; j < vd; j++) { Si[j] += ki * delta[j]; oh[j] += Si[j] * qi; }
        }
        /* gated RMSNorm (plain weight, not 1+w): qwen.c:353-357 */
        double ms = 0;
        for (int j = 0; j < vd; j++) ms += (double)oh[j] * oh[j];
        float r = 1.f / sqrtf((float)(ms / vd) + d->eps);
        const float *zh = z + h * vd;
        for (int j = 0; j < vd; j++) oh[j] = oh[j] * r * gnorm[j] * o_silu(zh[j]);
    }
    free(cv);
}

void gdno_core_seq(const gdno_dims *d, const float *conv_w, const float *A_log,
                   const float *dt_bias, const float *gnorm, int T,
                   const float *qkv, const float *z, const float *a, const float *b,
                   float *conv_st, float *S, float *core) {
    const int conv_dim = 2 * d->kh * d->kd + d->vh * d->vd, vdim = d->vh * d->vd;
    for (int t = 0; t < T; t++)
        gdno_core_step(d, conv_w, A_log, dt_bias, gnorm,
                       qkv + (int64_t)t * conv_dim, z + (int64_t)t * vdim,
                       a + (int64_t)t * d->vh, b + (int64_t)t * d->vh,
                       conv_st, S, core + (int64_t)t * vdim);
}

/* deltanet_step: qwen.c:301-364 (DM macro qwen.c:139-141 selects int8 twins). */
void gdno_layer_step(const gdno_dims *d, const gdno_layer_w *w, int int8,
                     const float *x, float *out, float *conv_st, float *S) {
    const int D = d->hidden, vh = d->vh;
    const int key_dim = d->kh * d->kd, val_dim = vh * d->vd, conv_dim = 2 * key_dim + val_dim;
    float *qkv = oalloc(conv_dim), *z = oalloc(val_dim), *bb = oalloc(vh), *aa = oalloc(vh);
    float *core = oalloc(val_dim);
    if (int8) gdno_matmul_q(qkv, x, w->Q_qkv, w->S_qkv, D, conv_dim);
    else      gdno_matvec(qkv, x, w->W_qkv, D, conv_dim);
    if (int8) gdno_matmul_q(z, x, w->Q_z, w->S_z, D, val_dim);
    else      gdno_matvec(z, x, w->W_z, D, val_dim);
    gdno_matvec(bb, x, w->W_b, D, vh);      /* b, a are fp32 in both modes (qwen.c:324-325) */
    gdno_matvec(aa, x, w->W_a, D, vh);
    gdno_core_step(d, w->conv_w, w->A_log, w->dt_bias, w->gnorm, qkv, z, aa, bb,
                   conv_st, S, core);
    if (int8) gdno_matmul_q(out, core, w->Q_out, w->S_out, val_dim, D);
    else      gdno_matvec(out, core, w->W_out, val_dim, D);
    free(qkv); free(z); free(bb); free(aa); free(core);
}

void gdno_layer_seq(const gdno_dims *d, const gdno_layer_w *w, int int8, int T,
                    const float *x, float *out, float *conv_st, float *S) {
    for (int t = 0; t < T; t++)
        gdno_layer_step(d, w, int8, x + (int64_t)t * d->hidden, out + (int64_t)t * d->hidden,
                        conv_st, S);
}

/* Chunked WY/UT form, transformers modeling_qwen3_5_moe.py:250-328, evaluated
 * in double.  One value head at a time; zero padding to a multiple of C
 * (TF:272-278) contributes g = 0 (no decay) and k = v = beta = 0. */
void gdno_chunked(int kh, int vh, int kd, int vd, int T, int C,
                  const float *q, const float *k, const float *v,
                  const float *g, const float *beta, float *S, float *o) {
    const int rep = vh / kh;
    const int nc = (T + C - 1) / C;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < vh; h++) {
        const int hk = h / rep;
        double *Sh = (double *)calloc((size_t)kd * vd, sizeof(double));
        double *gc = (double *)calloc(C, sizeof(double));
        double *A = (double *)calloc((size_t)C * C, sizeof(double));
        double *row = (double *)calloc(C, sizeof(double));
        double *U = (double *)calloc((size_t)C * vd, sizeof(double));
        double *W = (double *)calloc((size_t)C * kd, sizeof(double));
        double *vn = (double *)calloc((size_t)C * vd, sizeof(double));
        double *qc = (double *)calloc((size_t)C * kd, sizeof(double));
        double *kc = (double *)calloc((size_t)C * kd, sizeof(double));
        double *vc = (double *)calloc((size_t)C * vd, sizeof(double));
        double *bc = (double *)calloc(C, sizeof(double));
        for (int i = 0; i < kd * vd; i++) Sh[i] = S[(int64_t)h * kd * vd + i];
        for (int c = 0; c < nc; c++) {
            /* gather chunk (zero padded) */
            double run = 0;
            for (int t = 0; t < C; t++) {
                int tt = c * C + t;
                int live = tt < T;
                for (int i = 0; i < kd; i++) {
                    qc[t * kd + i] = live ? q[((int64_t)tt * kh + hk) * kd + i] : 0.0;
                    kc[t * kd + i] = live ? k[((int64_t)tt * kh + hk) * kd + i] : 0.0;
                }
                for (int j = 0; j < vd; j++) vc[t * vd + j] = live ? v[((int64_t)tt * vh + h) * vd + j] : 0.0;
                bc[t] = live ? beta[(int64_t)tt * vh + h] : 0.0;
                run += live ? g[(int64_t)tt * vh + h] : 0.0;
                gc[t] = run;
            }
            /* A = -(k_beta k^T ⊙ decay), strictly lower */
            for (int i = 0; i < C; i++)
                for (int j = 0; j < C; j++) {
                    double s = 0;
                    if (j < i) {
                        for (int e = 0; e < kd; e++) s += kc[i * kd + e] * kc[j * kd + e];
                        s = -(bc[i] * s) * exp(gc[i] - gc[j]);
                    }
                    A[i * C + j] = s;
                }
            /* forward substitution (TF:295-298), then + I */
            for (int i = 1; i < C; i++) {
                for (int j = 0; j < i; j++) row[j] = A[i * C + j];
                for (int j = 0; j < i; j++) {
                    double s = row[j];
                    for (int m = 0; m < i; m++) s += row[m] * A[m * C + j];
                    A[i * C + j] = s;
                }
            }
            for (int i = 0; i < C; i++) A[i * C + i] += 1.0;
            /* U = A (v*beta), W = A (k*beta*exp(gc)) */
            for (int i = 0; i < C; i++) {
                for (int j = 0; j < vd; j++) {
                    double s = 0;
                    for (int m = 0; m < C; m++) s += A[i * C + m] * vc[m * vd + j] * bc[m];
                    U[i * vd + j] = s;
                }
                for (int e = 0; e < kd; e++) {
                    double s = 0;
                    for (int m = 0; m < C; m++) s += A[i * C + m] * kc[m * kd + e] * bc[m] * exp(gc[m]);
                    W[i * kd + e] = s;
                }
            }
            /* v_new = U - W S */
            for (int i = 0; i < C; i++)
                for (int j = 0; j < vd; j++) {
                    double s = U[i * vd + j];
                    for (int e = 0; e < kd; e++) s -= W[i * kd + e] * Sh[e * vd + j];
                    vn[i * vd + j] = s;
                }
            /* o = (q*exp(gc)) S + (q k^T ⊙ decay, lower incl. diag) v_new */
            for (int i = 0; i < C; i++) {
                int tt = c * C + i;
                for (int j = 0; j < vd; j++) {
                    double s = 0;
                    for (int e = 0; e < kd; e++) s += qc[i * kd + e] * exp(gc[i]) * Sh[e * vd + j];
                    for (int m = 0; m <= i; m++) {
                        double qk = 0;
                        for (int e = 0; e < kd; e++) qk += qc[i * kd + e] * kc[m * kd + e];
                        s += qk * exp(gc[i] - gc[m]) * vn[m * vd + j];
                    }
                    if (tt < T) o[((int64_t)tt * vh + h) * vd + j] = (float)s;
                }
            }
            /* S = exp(g_last) S + (k * exp(g_last - gc))^T v_new */
            double gl = gc[C - 1];
            for (int e = 0; e < kd; e++)
                for (int j = 0; j < vd; j++) {
                    double s = Sh[e * vd + j] * exp(gl);
                    for (int m = 0; m < C; m++) s += kc[m * kd + e] * exp(gl - gc[m]) * vn[m * vd + j];
                    Sh[e * vd + j] = s;
                }
        }
        for (int i = 0; i < kd * vd; i++) S[(int64_t)h * kd * vd + i] = (float)Sh[i];
        free(Sh); free(gc); free(A); free(row); free(U); free(W); free(vn);
        free(qc); free(kc); free(vc); free(bc);
    }
}
