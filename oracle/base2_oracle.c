/*
 * CPU restatement of the integer ("all base 2") GPT-2 machine of base2.py.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only to check or to time the CPU side.  The product
 * path never calls it.
 *
 * Every operation follows the reference line it cites and reproduces numpy's
 * int64 behaviour exactly: additions and products wrap modulo 2^64, a left
 * shift by 64 or more gives 0, an arithmetic right shift by 64 or more gives
 * 0 or -1 (numpy's npy_lshift / npy_rshift guards).
 *
 * Two drivers are given:
 *   orc_forward  - base2.py:forward (base2.py:102-114): the whole sequence is
 *                  recomputed for the last position, as the reference does.
 *   orc_kv_step  - the same numbers for one new position with a per-layer
 *                  key/value cache (causality: every to16, gauge and arrival
 *                  acts on one row, so the cached step equals the recompute).
 *
 * Products are exact int64 sums.  base2.py forms them as float64 matrix
 * products guarded by |p| < 2^52 (base2.py:29-32); both agree whenever that
 * guard holds, and the same guard is reported here (return code ORC_E_BOUND).
 *
 * Parity pins: closed forms and brute force for each stage (tests/test_oracle_*),
 * golden vectors written by tests/golden/make_golden.py from base2.py itself.
 */
#include "orc_common.h"

/* base2.py:18-22  rshift(X, s): X x 2^-s rounded half up; s <= 0 is a left shift */
i64 orc_rshift1(i64 x, i64 s) {
    i64 up = shl(x, s < 0 ? -s : 0);
    i64 sp = s > 0 ? s : 0;
    i64 half = sp > 0 ? shl(1, sp - 1) : 0;
    return sar(wadd(up, half), sp);
}

/* base2.py:42-48  log2fix(v): top-1 position t, next 16 bits (truncated) into the LOG2 table */
i64 orc_log2fix1(i64 v, const i64* LOG2) {
    int t = bitlen_py(v) - 1;
    i64 m = t >= 16 ? (sar(v, t - 16) & 0xFFFF) : (shl(v, 16 - t) & 0xFFFF);
    return wadd(wmul((i64)t, 65536), LOG2[m]);
}

/* base2.py:50-53  power(X, F): X x 2^(F/65536) = rshift(X * EXP2[F & 0xFFFF], 16 - (F >> 16)) */
i64 orc_power1(i64 x, i64 F, const i64* EXP2) {
    i64 I = F >> 16, f = F & 0xFFFF;
    return orc_rshift1(wmul(x, EXP2[f]), wsub(16, I));
}

/* base2.py:24-27  to16 for one row: OR of |x|, sh = max(bitlen - 15, 0), x16 = rshift(x, sh) */
static int row_shift(const i64* x, i64 n) {
    i64 o = 0;
    for (i64 i = 0; i < n; i++) o |= iabs(x[i]);
    int top = bitlen_py(o);
    return top > 15 ? top - 15 : 0;
}
i64 orc_to16_row(const i64* x, i64 n, i64 e, i64* x16) {
    int sh = row_shift(x, n);
    for (i64 i = 0; i < n; i++) x16[i] = orc_rshift1(x[i], sh);
    return e + sh;
}

/* base2.py:34-40  race: the largest value, ties to the lowest index (the top-down bit elimination
 * over u = x ^ 2^63 keeps exactly the maximal values and then takes the first survivor) */
i64 orc_race(const i64* v, i64 n) {
    i64 best = 0;
    for (i64 i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}

/* base2.py:78-83  edge(H): share = PHI[rshift(H, 4) + 32768] (0 below, 65536 above); rshift(H * share, 16) */
i64 orc_edge1(i64 h, const i64* PHI) {
    i64 idx = wadd(orc_rshift1(h, 4), 32768);
    i64 share = idx < 0 ? 0 : (idx > 65535 ? 65536 : PHI[idx]);
    return orc_rshift1(wmul(h, share), 16);
}

/* ---------------- vector forms for the stage tests ---------------- */
/* OpenMP threads for the parallel loops below (the CPU baseline times one thread and all of them) */
#include <omp.h>
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : omp_get_num_procs()); }
int orc_get_threads(void) { return omp_get_max_threads(); }

void orc_rshift(const i64* x, const i64* s, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = orc_rshift1(x[i], s[i]); }
void orc_log2fix(const i64* v, i64* out, i64 n, const i64* LOG2) { for (i64 i = 0; i < n; i++) out[i] = orc_log2fix1(v[i], LOG2); }
void orc_power(const i64* x, const i64* F, i64* out, i64 n, const i64* EXP2) { for (i64 i = 0; i < n; i++) out[i] = orc_power1(x[i], F[i], EXP2); }
void orc_edge(const i64* h, i64* out, i64 n, const i64* PHI) { for (i64 i = 0; i < n; i++) out[i] = orc_edge1(h[i], PHI); }
void orc_to16(const i64* X, i64 rows, i64 n, i64 e, i64* x16, i64* ex) {
    for (i64 r = 0; r < rows; r++) ex[r] = orc_to16_row(X + r * n, n, e, x16 + r * n);
}

/* base2.py:55-60  gauge_log for one row of d values: x16, ex and LS (log2 of 1/sigma, units 2^-16) */
static i64 gauge_row(const i64* R, i64 d, i64* x16, i64* ex_out, i64 log768, i64 eps40, const i64* LOG2) {
    i64 ex = orc_to16_row(R, d, -16, x16);
    i64 s1 = 0, s2 = 0;
    for (i64 i = 0; i < d; i++) { s1 = wadd(s1, x16[i]); s2 = wadd(s2, wmul(x16[i], x16[i])); }
    i64 V = wsub(wmul(d, s2), wmul(s1, s1));
    i64 es = 40 + 2 * ex;            /* Python ints: EPS40 >> es, or << -es */
    i64 eps;
    if (es >= 0) eps = es >= 63 ? 0 : (eps40 >> es);
    else eps = shl(eps40, -es);
    V = wadd(V, eps);
    *ex_out = ex;
    return wadd(wsub(orc_log2fix1(V, LOG2) >> 1, log768), wmul(ex, 65536));
}
void orc_gauge_log(const i64* R, i64 rows, i64 d, i64* x16, i64* ex, i64* LS, i64 log768, i64 eps40, const i64* LOG2) {
    for (i64 r = 0; r < rows; r++) LS[r] = gauge_row(R + r * d, d, x16 + r * d, ex + r, log768, eps40, LOG2);
}

/* base2.py:29-32  product: exact sum of x16[i] * w[i][j] over a [nin][nout] int16 plate */
static int product_row(const i64* x16, i64 nin, const int16_t* w, i64 nout, i64* pile) {
    const i64 LIM = (i64)1 << 52;
    for (i64 j = 0; j < nout; j++) pile[j] = 0;
    for (i64 i = 0; i < nin; i++) {
        i64 xv = x16[i];
        if (!xv) continue;
        const int16_t* wr = w + i * nout;
        for (i64 j = 0; j < nout; j++) pile[j] += xv * (i64)wr[j];
    }
    int bad = 0;
    for (i64 j = 0; j < nout; j++) if (pile[j] >= LIM || pile[j] <= -LIM) bad = 1;
    return bad;
}
int orc_product(const i64* x16, i64 rows, i64 nin, const int16_t* w, i64 nout, i64* pile) {
    int bad = 0;
    #pragma omp parallel for schedule(static) reduction(|:bad)
    for (i64 r = 0; r < rows; r++) bad |= product_row(x16 + r * nin, nin, w, nout, pile + r * nout);
    return bad ? ORC_E_BOUND : ORC_OK;
}

/* ---------------- the model ---------------- */
typedef struct {
    int64_t n_layer, d, n_head, hd, d_ff, vocab, n_ctx;
    const int16_t* w[12][4];          /* qkv, proj, fc, mproj: [nin][nout] int16 (base2_convert.py layout) */
    const int64_t* e[12][4];
    const int64_t* b[12][4];
    const int16_t* head_w; const int64_t* head_e; const int64_t* head_b;
    const int64_t* wte; const int64_t* wpe;
    const int64_t* phi; const int64_t* arr; int64_t alen;
    const int64_t* log2t; const int64_t* exp2t;
    int64_t log768, eps40;
} orc_model;

/* per-position record of every intermediate (all int64); any pointer may be NULL */
typedef struct {
    int64_t* x16;     /* [L][4][3072]  light entering each bank (nin used) */
    int64_t* ex;      /* [L][4] */
    int64_t* ls;      /* [L][4]  gauge of the gauged banks (qkv, fc); 0 for plain banks */
    int64_t* pile;    /* [L][4][3072]  (nout used) */
    int64_t* qkv;     /* [L][2304] gauged qkv output */
    int64_t* att;     /* [L][768]  attention output */
    int64_t* hid;     /* [L][3072] fc output after the edge */
    int64_t* resid;   /* [L][2][768] stream after the attention half and after the MLP half */
    int64_t* head_x16; int64_t* head_ex; int64_t* head_ls;
    int64_t* head_pile; int64_t* logits;   /* [vocab] */
} orc_rec;

static const int NIN[4] = {768, 768, 768, 3072};
static const int NOUT[4] = {2304, 768, 3072, 768};

/* base2.py:62-71  gauged_bank for one row: power(pile, (we + ex + 16) * 65536 - LS) + b */
static int gauged_row(const orc_model* M, int l, int k, const i64* R, i64* out, i64* x16, i64* pile, i64* rex, i64* rls) {
    i64 ex, LS = gauge_row(R, M->d, x16, &ex, M->log768, M->eps40, M->log2t);
    int bad = product_row(x16, NIN[k], M->w[l][k], NOUT[k], pile);
    const i64* we = M->e[l][k]; const i64* b = M->b[l][k];
    for (int j = 0; j < NOUT[k]; j++)
        out[j] = wadd(orc_power1(pile[j], wsub(wmul(we[j] + ex + 16, 65536), LS), M->exp2t), b[j]);
    if (rex) *rex = ex;
    if (rls) *rls = LS;
    return bad;
}

/* base2.py:73-76  plain_bank for one row: rshift(pile, -(we + ex + 16)) + b, added onto the stream R */
static int plain_row_add(const orc_model* M, int l, int k, const i64* X, i64* R, i64* x16, i64* pile, i64* rex) {
    i64 ex = orc_to16_row(X, NIN[k], -16, x16);
    int bad = product_row(x16, NIN[k], M->w[l][k], NOUT[k], pile);
    const i64* we = M->e[l][k]; const i64* b = M->b[l][k];
    for (int j = 0; j < NOUT[k]; j++) R[j] = wadd(R[j], wadd(orc_rshift1(pile[j], -(we[j] + ex + 16)), b[j]));
    if (rex) *rex = ex;
    return bad;
}

/* one head's attention for the newest row p (base2.py:93-99):
 *   scores sc[s] = rshift(q16 . k16[s], -(eq + ek[s] - 3 + 10)), s <= p
 *   the clock starts at the maximum; a = ARR[max - sc] (0 past the table)
 *   out = power(sum a v, -log2fix(sum a)) with v the raw gauged value                 */
static int attend_row(const orc_model* M, const i64* q16, i64 eq, const i64* k16, const i64* ek, const i64* v,
                      i64 kstride, i64 vstride, i64 p, i64* sc, i64* out) {
    const i64 LIM = (i64)1 << 52;
    for (i64 s = 0; s <= p; s++) {
        i64 dot = 0;
        for (int t = 0; t < 64; t++) dot += q16[t] * k16[s * kstride + t];
        sc[s] = orc_rshift1(dot, -(eq + ek[s] - 3 + 10));
    }
    i64 best = sc[orc_race(sc, p + 1)];
    i64 Z = 0; i64 num[64] = {0};
    for (i64 s = 0; s <= p; s++) {
        i64 dd = wsub(best, sc[s]);
        i64 a = dd < M->alen ? M->arr[dd < M->alen - 1 ? dd : M->alen - 1] : 0;
        Z = wadd(Z, a);
        if (!a) continue;
        for (int t = 0; t < 64; t++) num[t] += a * v[s * vstride + t];
    }
    int bad = 0;
    i64 F = -orc_log2fix1(Z, M->log2t);
    for (int t = 0; t < 64; t++) {
        if (num[t] >= LIM || num[t] <= -LIM) bad = 1;
        out[t] = orc_power1(num[t], F, M->exp2t);
    }
    return bad;
}

/* base2.py:93-99 for the newest row p over a given cache (the device attention's contract, sm_stage_attend):
 * positions s < p from the caches k16 [12][ctx][64] (the keys' 16-bit lights), ek [12][ctx], v [12][ctx][64] (raw
 * values); position p from qkv [2304], its q and k through to16 (base2.py:93), its v raw.  out [768].  The same
 * attend_row as orc_attention, whose rows the golden vectors pin; a cache filled from QKV rows gives its rows. */
int orc_attend_cached(const orc_model* M, const i64* qkv, const i64* k16c, const i64* ekc, const i64* vc, i64 ctx,
                      i64 p, i64* out) {
    int bad = 0;
    i64* k16 = malloc(sizeof(i64) * (p + 1) * 64); i64* ek = malloc(sizeof(i64) * (p + 1));
    i64* v = malloc(sizeof(i64) * (p + 1) * 64); i64* sc = malloc(sizeof(i64) * (p + 1));
    for (int h = 0; h < 12; h++) {
        i64 q16[64];
        const i64 eq = orc_to16_row(qkv + h * 64, 64, -16, q16);
        for (i64 s = 0; s < p; s++) {
            memcpy(k16 + s * 64, k16c + (h * ctx + s) * 64, sizeof(i64) * 64);
            ek[s] = ekc[h * ctx + s];
            memcpy(v + s * 64, vc + (h * ctx + s) * 64, sizeof(i64) * 64);
        }
        ek[p] = orc_to16_row(qkv + 768 + h * 64, 64, -16, k16 + p * 64);
        memcpy(v + p * 64, qkv + 1536 + h * 64, sizeof(i64) * 64);
        bad |= attend_row(M, q16, eq, k16, ek, v, 64, 64, p, sc, out + h * 64);
    }
    free(k16); free(ek); free(v); free(sc);
    return bad ? ORC_E_BOUND : ORC_OK;
}

/* base2.py:85-100  attention over all P rows of QKV [P][2304] -> out [P][768] */
int orc_attention(const orc_model* M, const i64* QKV, i64 P, i64* out) {
    int bad = 0;
    #pragma omp parallel for schedule(dynamic) reduction(|:bad)
    for (int h = 0; h < 12; h++) {
        i64* q16 = malloc(sizeof(i64) * P * 64); i64* k16 = malloc(sizeof(i64) * P * 64);
        i64* eq = malloc(sizeof(i64) * P); i64* ek = malloc(sizeof(i64) * P);
        i64* v = malloc(sizeof(i64) * P * 64); i64* sc = malloc(sizeof(i64) * P);
        for (i64 p = 0; p < P; p++) {
            eq[p] = orc_to16_row(QKV + p * 2304 + h * 64, 64, -16, q16 + p * 64);
            ek[p] = orc_to16_row(QKV + p * 2304 + 768 + h * 64, 64, -16, k16 + p * 64);
            memcpy(v + p * 64, QKV + p * 2304 + 1536 + h * 64, sizeof(i64) * 64);
        }
        for (i64 p = 0; p < P; p++) bad |= attend_row(M, q16 + p * 64, eq[p], k16, ek, v, 64, 64, p, sc, out + p * 768 + h * 64);
        free(q16); free(k16); free(eq); free(ek); free(v); free(sc);
    }
    return bad ? ORC_E_BOUND : ORC_OK;
}

/* the head for one row (base2.py:107-114): gauge, product with head.w, power, + standing amount, race */
static int head_row(const orc_model* M, const i64* R, i64* logits, i64* x16, i64* pile, i64* rex, i64* rls, i64* token) {
    i64 ex, LS = gauge_row(R, M->d, x16, &ex, M->log768, M->eps40, M->log2t);
    int bad = 0;
    const i64 V = M->vocab;
    i64* part = pile;
    for (i64 j = 0; j < V; j++) part[j] = 0;
    /* exact product over the 768 x V plate, split over threads by columns */
    #pragma omp parallel for schedule(static)
    for (i64 j0 = 0; j0 < V; j0 += 4096) {
        i64 j1 = j0 + 4096 < V ? j0 + 4096 : V;
        for (i64 i = 0; i < M->d; i++) {
            i64 xv = x16[i]; if (!xv) continue;
            const int16_t* wr = M->head_w + i * V;
            for (i64 j = j0; j < j1; j++) part[j] += xv * (i64)wr[j];
        }
    }
    const i64 LIM = (i64)1 << 52;
    for (i64 j = 0; j < V; j++) {
        if (part[j] >= LIM || part[j] <= -LIM) bad = 1;
        logits[j] = wadd(orc_power1(part[j], wsub(wmul(M->head_e[j] + ex + 16, 65536), LS), M->exp2t), M->head_b[j]);
    }
    *token = orc_race(logits, V);
    if (rex) *rex = ex;
    if (rls) *rls = LS;
    return bad;
}

#define RX(p, l, k) ((p) + ((l) * 4 + (k)) * 3072)
#define R1(p, l, k) ((p) + (l) * 4 + (k))

/* base2.py:102-114  forward(ids): full recompute of all P positions; returns the next word
 * (>= 0) or a negative error.  rec (optional) receives the last position's intermediates. */
int64_t orc_forward(const orc_model* M, const int32_t* ids, i64 P, orc_rec* rec, int* status) {
    const i64 D = M->d;
    i64* R = malloc(sizeof(i64) * P * D);
    i64* QKV = malloc(sizeof(i64) * P * 2304);
    i64* att = malloc(sizeof(i64) * P * 768);
    i64* hid = malloc(sizeof(i64) * P * 3072);
    i64* x16 = malloc(sizeof(i64) * P * 3072);
    i64* pile = malloc(sizeof(i64) * P * (M->vocab > 3072 ? M->vocab : 3072));
    int bad = 0;
    for (i64 p = 0; p < P; p++)
        for (i64 i = 0; i < D; i++) R[p * D + i] = wadd(M->wte[(i64)ids[p] * D + i], M->wpe[p * D + i]);
    for (int l = 0; l < 12; l++) {
        i64 ex[4], ls[4];
        #pragma omp parallel for schedule(static) reduction(|:bad)
        for (i64 p = 0; p < P; p++)
            bad |= gauged_row(M, l, 0, R + p * D, QKV + p * 2304, x16 + p * 3072, pile + p * 3072,
                              p == P - 1 ? &ex[0] : NULL, p == P - 1 ? &ls[0] : NULL);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 0), x16 + (P - 1) * 3072, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 0), pile + (P - 1) * 3072, sizeof(i64) * 2304);
            if (rec->qkv) memcpy(rec->qkv + l * 2304, QKV + (P - 1) * 2304, sizeof(i64) * 2304);
        }
        bad |= orc_attention(M, QKV, P, att);
        if (rec && rec->att) memcpy(rec->att + l * 768, att + (P - 1) * 768, sizeof(i64) * 768);
        #pragma omp parallel for schedule(static) reduction(|:bad)
        for (i64 p = 0; p < P; p++)
            bad |= plain_row_add(M, l, 1, att + p * 768, R + p * D, x16 + p * 3072, pile + p * 3072, p == P - 1 ? &ex[1] : NULL);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 1), x16 + (P - 1) * 3072, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 1), pile + (P - 1) * 3072, sizeof(i64) * 768);
            if (rec->resid) memcpy(rec->resid + (l * 2) * 768, R + (P - 1) * D, sizeof(i64) * 768);
        }
        #pragma omp parallel for schedule(static) reduction(|:bad)
        for (i64 p = 0; p < P; p++) {
            bad |= gauged_row(M, l, 2, R + p * D, hid + p * 3072, x16 + p * 3072, pile + p * 3072,
                              p == P - 1 ? &ex[2] : NULL, p == P - 1 ? &ls[2] : NULL);
            for (int j = 0; j < 3072; j++) hid[p * 3072 + j] = orc_edge1(hid[p * 3072 + j], M->phi);
        }
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 2), x16 + (P - 1) * 3072, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 2), pile + (P - 1) * 3072, sizeof(i64) * 3072);
            if (rec->hid) memcpy(rec->hid + l * 3072, hid + (P - 1) * 3072, sizeof(i64) * 3072);
        }
        #pragma omp parallel for schedule(static) reduction(|:bad)
        for (i64 p = 0; p < P; p++)
            bad |= plain_row_add(M, l, 3, hid + p * 3072, R + p * D, x16 + p * 3072, pile + p * 3072, p == P - 1 ? &ex[3] : NULL);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 3), x16 + (P - 1) * 3072, sizeof(i64) * 3072);
            if (rec->pile) memcpy(RX(rec->pile, l, 3), pile + (P - 1) * 3072, sizeof(i64) * 768);
            if (rec->resid) memcpy(rec->resid + (l * 2 + 1) * 768, R + (P - 1) * D, sizeof(i64) * 768);
            ls[1] = ls[3] = 0;
            for (int k = 0; k < 4; k++) { if (rec->ex) *R1(rec->ex, l, k) = ex[k]; if (rec->ls) *R1(rec->ls, l, k) = ls[k]; }
        }
    }
    i64 tok, hex, hls;
    i64* logits = malloc(sizeof(i64) * M->vocab);
    bad |= head_row(M, R + (P - 1) * D, logits, x16, pile, &hex, &hls, &tok);
    if (rec) {
        if (rec->head_x16) memcpy(rec->head_x16, x16, sizeof(i64) * 768);
        if (rec->head_ex) *rec->head_ex = hex;
        if (rec->head_ls) *rec->head_ls = hls;
        if (rec->head_pile) memcpy(rec->head_pile, pile, sizeof(i64) * M->vocab);
        if (rec->logits) memcpy(rec->logits, logits, sizeof(i64) * M->vocab);
    }
    free(R); free(QKV); free(att); free(hid); free(x16); free(pile); free(logits);
    if (status) *status = bad ? ORC_E_BOUND : ORC_OK;
    return tok;
}

/* ---------------- KV-cached machine (one new position per call) ---------------- */
typedef struct {
    int64_t max_ctx, pos;
    int64_t* k16;   /* [L][ctx][768] per-head 16-bit keys */
    int64_t* ek;    /* [L][ctx][12] */
    int64_t* v;     /* [L][ctx][768] raw gauged values */
    int64_t* R;     /* [768] */
} orc_kv;

orc_kv* orc_kv_new(int64_t max_ctx) {
    orc_kv* S = calloc(1, sizeof(orc_kv));
    S->max_ctx = max_ctx;
    S->k16 = calloc((size_t)12 * max_ctx * 768, sizeof(i64));
    S->ek = calloc((size_t)12 * max_ctx * 12, sizeof(i64));
    S->v = calloc((size_t)12 * max_ctx * 768, sizeof(i64));
    S->R = calloc(768, sizeof(i64));
    return S;
}
void orc_kv_free(orc_kv* S) { if (!S) return; free(S->k16); free(S->ek); free(S->v); free(S->R); free(S); }
int64_t orc_kv_pos(const orc_kv* S) { return S->pos; }

/* one new position: token `tok` enters at S->pos; returns the next word (the race at the top) when
 * want_head != 0, else -1.  Intermediates of this position go to rec (optional). */
int64_t orc_kv_step(const orc_model* M, orc_kv* S, int32_t tok, int want_head, orc_rec* rec, int* status) {
    if (S->pos >= S->max_ctx || tok < 0 || tok >= M->vocab) { if (status) *status = ORC_E_ARG; return -1; }
    const i64 D = M->d, p = S->pos;
    i64* R = S->R;
    i64 qkv[2304], att[768], hid[3072], x16[3072], pile[3072];
    i64* sc = malloc(sizeof(i64) * (p + 1));
    int bad = 0;
    for (i64 i = 0; i < D; i++) R[i] = wadd(M->wte[(i64)tok * D + i], M->wpe[p * D + i]);
    for (int l = 0; l < 12; l++) {
        i64 ex[4] = {0}, ls[4] = {0};
        bad |= gauged_row(M, l, 0, R, qkv, x16, pile, &ex[0], &ls[0]);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 0), x16, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 0), pile, sizeof(i64) * 2304);
            if (rec->qkv) memcpy(rec->qkv + l * 2304, qkv, sizeof(i64) * 2304);
        }
        i64* K = S->k16 + (size_t)l * S->max_ctx * 768;
        i64* EK = S->ek + (size_t)l * S->max_ctx * 12;
        i64* VV = S->v + (size_t)l * S->max_ctx * 768;
        for (int h = 0; h < 12; h++) {
            EK[p * 12 + h] = orc_to16_row(qkv + 768 + h * 64, 64, -16, K + p * 768 + h * 64);
            memcpy(VV + p * 768 + h * 64, qkv + 1536 + h * 64, sizeof(i64) * 64);
        }
        for (int h = 0; h < 12; h++) {
            i64 q16[64];
            i64 eq = orc_to16_row(qkv + h * 64, 64, -16, q16);
            /* ek for head h at every cached position */
            i64* ekc = malloc(sizeof(i64) * (p + 1));
            for (i64 s = 0; s <= p; s++) ekc[s] = EK[s * 12 + h];
            bad |= attend_row(M, q16, eq, K + h * 64, ekc, VV + h * 64, 768, 768, p, sc, att + h * 64);
            free(ekc);
        }
        if (rec && rec->att) memcpy(rec->att + l * 768, att, sizeof(i64) * 768);
        bad |= plain_row_add(M, l, 1, att, R, x16, pile, &ex[1]);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 1), x16, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 1), pile, sizeof(i64) * 768);
            if (rec->resid) memcpy(rec->resid + (l * 2) * 768, R, sizeof(i64) * 768);
        }
        bad |= gauged_row(M, l, 2, R, hid, x16, pile, &ex[2], &ls[2]);
        for (int j = 0; j < 3072; j++) hid[j] = orc_edge1(hid[j], M->phi);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 2), x16, sizeof(i64) * 768);
            if (rec->pile) memcpy(RX(rec->pile, l, 2), pile, sizeof(i64) * 3072);
            if (rec->hid) memcpy(rec->hid + l * 3072, hid, sizeof(i64) * 3072);
        }
        bad |= plain_row_add(M, l, 3, hid, R, x16, pile, &ex[3]);
        if (rec) {
            if (rec->x16) memcpy(RX(rec->x16, l, 3), x16, sizeof(i64) * 3072);
            if (rec->pile) memcpy(RX(rec->pile, l, 3), pile, sizeof(i64) * 768);
            if (rec->resid) memcpy(rec->resid + (l * 2 + 1) * 768, R, sizeof(i64) * 768);
            for (int k = 0; k < 4; k++) { if (rec->ex) *R1(rec->ex, l, k) = ex[k]; if (rec->ls) *R1(rec->ls, l, k) = ls[k]; }
        }
    }
    free(sc);
    S->pos++;
    i64 tokn = -1;
    if (want_head) {
        i64 hex, hls;
        i64* logits = malloc(sizeof(i64) * M->vocab);
        i64* hp = malloc(sizeof(i64) * M->vocab);
        bad |= head_row(M, R, logits, x16, hp, &hex, &hls, &tokn);
        if (rec) {
            if (rec->head_x16) memcpy(rec->head_x16, x16, sizeof(i64) * 768);
            if (rec->head_ex) *rec->head_ex = hex;
            if (rec->head_ls) *rec->head_ls = hls;
            if (rec->head_pile) memcpy(rec->head_pile, hp, sizeof(i64) * M->vocab);
            if (rec->logits) memcpy(rec->logits, logits, sizeof(i64) * M->vocab);
        }
        free(logits); free(hp);
    }
    if (status) *status = bad ? ORC_E_BOUND : ORC_OK;
    return tokn;
}

/* read back the cache of one layer at one position: k16 [768], ek [12], v [768] */
void orc_kv_read(const orc_kv* S, int64_t layer, int64_t pos, int64_t* k16, int64_t* ek, int64_t* v) {
    if (k16) memcpy(k16, S->k16 + ((size_t)layer * S->max_ctx + pos) * 768, sizeof(i64) * 768);
    if (ek) memcpy(ek, S->ek + ((size_t)layer * S->max_ctx + pos) * 12, sizeof(i64) * 12);
    if (v) memcpy(v, S->v + ((size_t)layer * S->max_ctx + pos) * 768, sizeof(i64) * 768);
}
void orc_kv_read_resid(const orc_kv* S, int64_t* R) { memcpy(R, S->R, sizeof(i64) * 768); }
