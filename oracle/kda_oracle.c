/*
 * kda_oracle.c -- plain-C fp64 restatement of the reference's KDA step
 * recurrence.  TEST INFRASTRUCTURE ONLY: linked by tests/, smoke() and the
 * bench's cpu_baseline leg as the checker, never by the product library.
 *
 * Forward (per (b, h), one token at a time), the rank-1 form of the step in
 * nope_gdn_mlx.py:616-638 given at nope_gdn_mlx.py:3724-3735 and used by the
 * Metal kernel at nope_gdn_mlx.py:3003-3019:
 *     S'  = S diag(exp(g_t))            column scale, columns = key channels
 *     u   = beta_t (v_t - S' k_t)
 *     S   = S' + u k_t^T
 *     o_t = S q_t                       post-update state
 * State layout S[b][h][i_v][j_k] (reference orientation).
 *
 * Backward: the reverse-time adjoint of nope_gdn_mlx.py:3185-3295
 * (_kda_python_backward_full).  States are re-materialised from checkpoints
 * taken every KDA_ORACLE_CKPT steps instead of keeping all L+1 of them.
 *
 * Tensors are contiguous: q/k/v/g/o and their grads (B, T, H, D); beta and
 * dbeta (B, T, H); states (B, H, D, D).  Work is split over (b, h) across
 * `nthreads` pthreads.  Return value: 0 on success, -1 on bad arguments,
 * -2 on allocation failure.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define KDA_ORACLE_CKPT 64

typedef struct {
    const double *q, *k, *v, *g, *beta, *s0, *dout, *dsf;
    double *o, *sf, *dq, *dk, *dv, *dg, *dbeta, *ds0;
    int B, T, H, D, backward;
    int next;
    int err;
    pthread_mutex_t mu;
} kda_job;

static inline size_t vidx(const kda_job *J, int b, int t, int h) {
    return (((size_t)b * J->T + t) * J->H + h) * (size_t)J->D;
}
static inline size_t sidx(const kda_job *J, int b, int t, int h) {
    return ((size_t)b * J->T + t) * J->H + h;
}

/* One forward step on state S (D x D); writes u (D) and, if o != NULL, o (D). */
static void step_fwd(int D, double *S, const double *qt, const double *kt, const double *vt,
                     const double *gt, double bt, double *u, double *o, double *dec) {
    for (int j = 0; j < D; ++j) dec[j] = exp(gt[j]);
    for (int i = 0; i < D; ++i) {
        double *row = S + (size_t)i * D;
        double sk = 0.0;
        for (int j = 0; j < D; ++j) { row[j] *= dec[j]; sk += row[j] * kt[j]; }
        u[i] = bt * (vt[i] - sk);
    }
    for (int i = 0; i < D; ++i) {
        double *row = S + (size_t)i * D;
        double acc = 0.0;
        for (int j = 0; j < D; ++j) { row[j] += u[i] * kt[j]; acc += row[j] * (qt ? qt[j] : 0.0); }
        if (o) o[i] = acc;
    }
}

static int run_forward(kda_job *J, int b, int h) {
    const int D = J->D, T = J->T;
    double *S = (double *)malloc(sizeof(double) * ((size_t)D * D + 2 * (size_t)D));
    if (!S) return -2;
    double *u = S + (size_t)D * D, *dec = u + D;
    if (J->s0) memcpy(S, J->s0 + ((size_t)b * J->H + h) * D * D, sizeof(double) * D * D);
    else memset(S, 0, sizeof(double) * D * D);
    for (int t = 0; t < T; ++t) {
        size_t x = vidx(J, b, t, h);
        step_fwd(D, S, J->q + x, J->k + x, J->v + x, J->g + x, J->beta[sidx(J, b, t, h)], u,
                 J->o + x, dec);
    }
    if (J->sf) memcpy(J->sf + ((size_t)b * J->H + h) * D * D, S, sizeof(double) * D * D);
    free(S);
    return 0;
}

static int run_backward(kda_job *J, int b, int h) {
    const int D = J->D, T = J->T, CK = KDA_ORACLE_CKPT;
    const size_t DD = (size_t)D * D;
    const int nck = (T + CK - 1) / CK;
    /* checkpoints: state before step c*CK; segment buffer: state before each step */
    double *ck = (double *)malloc(sizeof(double) * DD * (size_t)(nck > 0 ? nck : 1));
    double *seg = (double *)malloc(sizeof(double) * DD * CK);
    double *work = (double *)malloc(sizeof(double) * (3 * DD + 10 * (size_t)D));
    if (!ck || !seg || !work) { free(ck); free(seg); free(work); return -2; }
    double *Sp = work, *St = Sp + DD, *gS = St + DD;
    double *u = gS + DD, *w = u + D, *dec = w + D, *du = dec + D, *dw = du + D;

    double *S = St;
    if (J->s0) memcpy(S, J->s0 + ((size_t)b * J->H + h) * DD, sizeof(double) * DD);
    else memset(S, 0, sizeof(double) * DD);
    for (int t = 0; t < T; ++t) {
        if (t % CK == 0) memcpy(ck + (size_t)(t / CK) * DD, S, sizeof(double) * DD);
        size_t x = vidx(J, b, t, h);
        step_fwd(D, S, NULL, J->k + x, J->v + x, J->g + x, J->beta[sidx(J, b, t, h)], u, NULL, dec);
    }
    if (J->dsf) memcpy(gS, J->dsf + ((size_t)b * J->H + h) * DD, sizeof(double) * DD);
    else memset(gS, 0, sizeof(double) * DD);

    for (int c = nck - 1; c >= 0; --c) {
        const int t0 = c * CK, t1 = (t0 + CK < T) ? t0 + CK : T;
        memcpy(St, ck + (size_t)c * DD, sizeof(double) * DD);
        for (int t = t0; t < t1; ++t) {
            memcpy(seg + (size_t)(t - t0) * DD, St, sizeof(double) * DD);
            size_t x = vidx(J, b, t, h);
            step_fwd(D, St, NULL, J->k + x, J->v + x, J->g + x, J->beta[sidx(J, b, t, h)], u, NULL, dec);
        }
        for (int t = t1 - 1; t >= t0; --t) {
            const size_t x = vidx(J, b, t, h);
            const double *qt = J->q + x, *kt = J->k + x, *vt = J->v + x, *gt = J->g + x;
            const double *dot = J->dout + x;
            const double bt = J->beta[sidx(J, b, t, h)];
            const double *Sprev = seg + (size_t)(t - t0) * DD;
            /* S' = Sprev diag(e^g);  w = v - S'k;  u = beta w;  S_t = S' + u k^T */
            for (int j = 0; j < D; ++j) dec[j] = exp(gt[j]);
            for (int i = 0; i < D; ++i) {
                double sk = 0.0;
                for (int j = 0; j < D; ++j) {
                    double s = Sprev[(size_t)i * D + j] * dec[j];
                    Sp[(size_t)i * D + j] = s;
                    sk += s * kt[j];
                }
                w[i] = vt[i] - sk;
                u[i] = bt * w[i];
            }
            /* gS += do q^T */
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) gS[(size_t)i * D + j] += dot[i] * qt[j];
            /* dq = S_t^T do = S'^T do + k (u . do) */
            double ud = 0.0;
            for (int i = 0; i < D; ++i) ud += u[i] * dot[i];
            for (int j = 0; j < D; ++j) {
                double acc = 0.0;
                for (int i = 0; i < D; ++i) acc += Sp[(size_t)i * D + j] * dot[i];
                J->dq[x + j] = acc + kt[j] * ud;
            }
            /* du = gS k; dbeta = du . w; dw = beta du = dv */
            double dbeta = 0.0;
            for (int i = 0; i < D; ++i) {
                double acc = 0.0;
                for (int j = 0; j < D; ++j) acc += gS[(size_t)i * D + j] * kt[j];
                du[i] = acc;
                dbeta += acc * w[i];
                dw[i] = bt * acc;
                J->dv[x + i] = dw[i];
            }
            J->dbeta[sidx(J, b, t, h)] = dbeta;
            /* dk = gS^T u - S'^T dw;  dS' = gS - dw k^T;  dg = colsum(dS' . S') */
            for (int j = 0; j < D; ++j) {
                double a = 0.0, bsum = 0.0, gsum = 0.0;
                for (int i = 0; i < D; ++i) {
                    const double gs = gS[(size_t)i * D + j];
                    const double sp = Sp[(size_t)i * D + j];
                    a += gs * u[i];
                    bsum += sp * dw[i];
                    gsum += (gs - dw[i] * kt[j]) * sp;
                }
                J->dk[x + j] = a - bsum;
                J->dg[x + j] = gsum;
            }
            /* gS <- dS' diag(e^g) */
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    double *p = gS + (size_t)i * D + j;
                    *p = (*p - dw[i] * kt[j]) * dec[j];
                }
        }
    }
    if (J->ds0) memcpy(J->ds0 + ((size_t)b * J->H + h) * DD, gS, sizeof(double) * DD);
    free(ck); free(seg); free(work);
    return 0;
}

static void *worker(void *arg) {
    kda_job *J = (kda_job *)arg;
    for (;;) {
        pthread_mutex_lock(&J->mu);
        int bh = J->next++;
        pthread_mutex_unlock(&J->mu);
        if (bh >= J->B * J->H) break;
        int rc = J->backward ? run_backward(J, bh / J->H, bh % J->H)
                             : run_forward(J, bh / J->H, bh % J->H);
        if (rc) {
            pthread_mutex_lock(&J->mu);
            J->err = rc;
            pthread_mutex_unlock(&J->mu);
        }
    }
    return NULL;
}

static int run_job(kda_job *J, int nthreads) {
    if (J->B < 0 || J->T < 0 || J->H < 0 || J->D <= 0) return -1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    J->next = 0;
    J->err = 0;
    pthread_mutex_init(&J->mu, NULL);
    pthread_t th[256];
    int started = 0;
    for (int i = 0; i < nthreads; ++i)
        if (pthread_create(&th[i], NULL, worker, J) == 0) ++started;
    if (started == 0) worker(J);
    for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
    pthread_mutex_destroy(&J->mu);
    return J->err;
}

int kda_oracle_fwd(const double *q, const double *k, const double *v, const double *g,
                   const double *beta, const double *s0, double *o, double *s_final,
                   int B, int T, int H, int D, int nthreads) {
    if (!q || !k || !v || !g || !beta || !o) return -1;
    kda_job J;
    memset(&J, 0, sizeof(J));
    J.q = q; J.k = k; J.v = v; J.g = g; J.beta = beta; J.s0 = s0;
    J.o = o; J.sf = s_final;
    J.B = B; J.T = T; J.H = H; J.D = D; J.backward = 0;
    return run_job(&J, nthreads);
}

int kda_oracle_bwd(const double *q, const double *k, const double *v, const double *g,
                   const double *beta, const double *s0, const double *dout,
                   const double *ds_final, double *dq, double *dk, double *dv, double *dg,
                   double *dbeta, double *ds0, int B, int T, int H, int D, int nthreads) {
    if (!q || !k || !v || !g || !beta || !dout || !dq || !dk || !dv || !dg || !dbeta) return -1;
    kda_job J;
    memset(&J, 0, sizeof(J));
    J.q = q; J.k = k; J.v = v; J.g = g; J.beta = beta; J.s0 = s0;
    J.dout = dout; J.dsf = ds_final;
    J.dq = dq; J.dk = dk; J.dv = dv; J.dg = dg; J.dbeta = dbeta; J.ds0 = ds0;
    J.B = B; J.T = T; J.H = H; J.D = D; J.backward = 1;
    return run_job(&J, nthreads);
}
