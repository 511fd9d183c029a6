/*
 * CPU restatement of the Pythia-shaped integer machine of foundation0/pythia_base2.py.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP library: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The product path never calls it.
 *
 * It follows pythia_base2.py with plates=finished, order=plain and every stage switch "int":
 *   embed    R = rshift(embed.w[id], -(embed.e[id] + 16))                          (pythia_base2.py:153)
 *   gauge    x16, ex = to16(R); S1, S2; c = d x16 - S1; V = d S2 - S1^2 + EPS40 >> (40 + 2 ex);
 *            LS = log2fix(V) >> 1; power(c g, (ge + 16) 65536 - LS) + b               (:100-110)
 *   plain    rshift(product(to16(X)), -(e + ex + 16)) + b, every plate                (:112-114)
 *   turn     the first ROT dims of q and k: pairs (i, i + ROT/2) by COS/SIN[pos] at 2^-30 (:116-123)
 *   attend   per head h: q, k, v at h*3*HS (interleaved); scores power(q16.k16, (eq + ek + 10) 65536 - HALF);
 *            the level = max; a = ARR[level - sc] (0 past the table); power(a.v, -log2fix(sum a))  (:125-141)
 *   edge     as base2.py (rshift(H, 4) + 32768 into PHI, rshift(H share, 16))         (:143-147)
 *   layer    R = R + plain(attend(plain(gauge(R, ln1), qkv)), proj) + plain(edge(plain(gauge(R, ln2), fc)), mproj)
 *   head     y16, ey = to16(gauge(R, lnf)); rshift(product(y16, head.w), -(head.e + ey + 16)); race  (:158-160)
 * power is exact here (pythia_base2.py:87-90 takes int64 when every |X| < 2^45 and Python integers beyond, so it
 * never wraps): X * EXP2[f] is formed in 128 bits.  The reference's asserts come back as status codes; they are
 * checked per element (the reference checks the largest element of the array against the smallest shift).
 * Additions onto the stream, the edge's product and the turns' products are numpy int64 operations (they wrap).
 *
 * Parity pins: the golden vectors of tests/golden/make_golden_pythia.py (words and every intermediate of the last
 * position, written by executing pythia_base2.py itself on the same converted arrays) and the attention goldens.
 */
#include "orc_common.h"

#define PYO_E_SHIFT 3     /* rshift: a left shift past 2^62 (pythia_base2.py:63) */
#define PYO_E_TURN 4      /* turn: |X| >= 2^31 in the turned dims (:121) */
#define PYO_E_ATT 5       /* attention: max|v| sum(a) >= 2^62 (:138) */
#define PYO_E_POW 6       /* power: the exact result does not fit int64 (:85) */

typedef __int128 i128;

typedef struct {
    int64_t L, d, heads, hs, rot, vocab, npos, alen;
    const int16_t* w[12][4]; const int64_t* e[12][4]; const int64_t* b[12][4];   /* [nin][nout] plates */
    const int64_t* ng[12][2]; int64_t nge[12][2]; const int64_t* nb[12][2];      /* ln1, ln2 gain, power, offset */
    const int64_t* fg; int64_t fge; const int64_t* fb;                             /* lnf */
    const int16_t* hw; const int64_t* he;                                          /* head [d][vocab], power per word */
    const int16_t* ew; const int64_t* ee;                                          /* embed [vocab][d], power per word */
    const int64_t* phi; const int64_t* arr; const int64_t* log2t; const int64_t* exp2t;
    const int64_t* cosT; const int64_t* sinT;                                      /* [npos][rot / 2] at 2^-30 */
    int64_t eps40, half;
    double wmax[12][4], hwmax;                                                     /* filled by pyo_prepare */
} py_model;

typedef struct {                   /* one position's intermediates; any pointer may be NULL */
    int64_t* stream;               /* [L][768] the stream entering each layer */
    int64_t* g1; int64_t* g2;      /* [L][768] the two gauges */
    int64_t* x16; int64_t* ex;     /* [L][4][3072], [L][4]: each plate's light and water level */
    int64_t* pile; int64_t* out;   /* [L][4][3072] */
    int64_t* att; int64_t* hid;    /* [L][768], [L][3072] */
    int64_t* stream_final; int64_t* glnf; int64_t* hx16; int64_t* hex; int64_t* hpile; int64_t* logits;
} py_rec;

static const int PNIN[4] = {768, 768, 768, 3072};
static const int PNOUT[4] = {2304, 768, 3072, 768};

static void flag(int* st, int code) { if (!*st) *st = code; }

/* pythia_base2.py:61-65  rshift with the left-shift bound of :63 */
static i64 prsh(i64 x, i64 s, int* st) {
    if (s < 0 && (62 + s <= 0 || iabs(x) >= ((i64)1 << (62 + s)))) flag(st, PYO_E_SHIFT);
    return orc_rshift1(x, s);
}

/* pythia_base2.py:87-90  power(X, F) = X x 2^(F/65536), exact */
static i64 ppow(i64 x, i64 F, const i64* EXP2, int* st) {
    const i64 I = F >> 16, f = F & 0xFFFF;
    const i128 X = (i128)x * EXP2[f];
    const i64 s = 16 - I;
    i128 r;
    if (s <= 0) {
        const i128 ax = X < 0 ? -X : X;
        if (X != 0 && (-s > 62 || ax >= ((i128)1 << (63 + s)))) { flag(st, PYO_E_POW); return 0; }
        r = X << -s;
    } else if (s >= 100) {
        r = 0;                                      /* |X| < 2^81: (X + 2^(s-1)) >> s is 0 */
    } else {
        r = (X + ((i128)1 << (s - 1))) >> s;
    }
    if (r > (i128)INT64_MAX || r < (i128)INT64_MIN) { flag(st, PYO_E_POW); return 0; }
    return (i64)r;
}

/* pythia_base2.py:74-80  product: exact sums; the assert sum|x16| max|w| < 2^53 */
static void pprod(const i64* x16, i64 nin, const int16_t* w, i64 nout, double wmax, i64* pile, int* st) {
    double sa = 0;
    for (i64 i = 0; i < nin; i++) sa += (double)iabs(x16[i]);
    if (sa * wmax >= 9007199254740992.0) flag(st, ORC_E_BOUND);
    #pragma omp parallel for schedule(static)
    for (i64 j0 = 0; j0 < nout; j0 += 1024) {
        const i64 j1 = j0 + 1024 < nout ? j0 + 1024 : nout;
        for (i64 j = j0; j < j1; j++) pile[j] = 0;
        for (i64 i = 0; i < nin; i++) {
            const i64 xv = x16[i];
            if (!xv) continue;
            const int16_t* wr = w + i * nout;
            for (i64 j = j0; j < j1; j++) pile[j] += xv * (i64)wr[j];
        }
    }
}

/* pythia_base2.py:100-110  the gauge of one row */
static void pgauge(const py_model* M, const i64* R, const i64* g, i64 ge, const i64* b, i64* out, int* st) {
    const i64 d = M->d;
    i64 x16[768];
    const i64 ex = orc_to16_row(R, d, -16, x16);
    i64 S1 = 0, S2 = 0;
    for (i64 i = 0; i < d; i++) { S1 = wadd(S1, x16[i]); S2 = wadd(S2, wmul(x16[i], x16[i])); }
    const i64 es = 40 + 2 * ex;                     /* ex >= -16: es >= 8 */
    const i64 V = wadd(wsub(wmul(d, S2), wmul(S1, S1)), es >= 63 ? 0 : (M->eps40 >> es));
    const i64 LS = orc_log2fix1(V, M->log2t) >> 1;
    const i64 F = wsub(wmul(ge + 16, 65536), LS);
    for (i64 i = 0; i < d; i++) {
        const i64 c = wsub(wmul(d, x16[i]), S1);
        out[i] = wadd(ppow(wmul(c, g[i]), F, M->exp2t, st), b[i]);
    }
}

/* pythia_base2.py:112-114  plain plate of one row (b may be NULL: the head) */
static i64 pplain(const int16_t* w, const i64* e, const i64* b, double wmax, const i64* X, i64 nin, i64 nout,
                  i64* out, i64* x16, i64* pile, int* st) {
    const i64 ex = orc_to16_row(X, nin, -16, x16);
    pprod(x16, nin, w, nout, wmax, pile, st);
    for (i64 j = 0; j < nout; j++) {
        const i64 y = prsh(pile[j], -(e[j] + ex + 16), st);
        out[j] = b ? wadd(y, b[j]) : y;
    }
    return ex;
}

/* pythia_base2.py:116-123  the turns of one head's q or k at position pos */
static void pturn(const py_model* M, i64* x, i64 pos, int* st) {
    const i64 r = M->rot / 2;
    for (i64 i = 0; i < M->rot; i++) if (iabs(x[i]) >= ((i64)1 << 31)) flag(st, PYO_E_TURN);
    const i64* c = M->cosT + pos * r;
    const i64* s = M->sinT + pos * r;
    for (i64 i = 0; i < r; i++) {
        const i64 a = x[i], bb = x[i + r];
        x[i] = prsh(wsub(wmul(a, c[i]), wmul(bb, s[i])), 30, st);
        x[i + r] = prsh(wadd(wmul(bb, c[i]), wmul(a, s[i])), 30, st);
    }
}

/* one layer's attention for the newest position p, given its QKV row; the caches receive position p:
 * K16 [ctx][d] (to16 of the turned keys), EK [ctx][heads], V [ctx][d] (raw values) */
static void pattend(const py_model* M, const i64* qkv, i64 p, i64* K16, i64* EK, i64* V, i64* sc, i64* out, int* st) {
    const i64 d = M->d, H = M->heads, HS = M->hs;
    for (i64 h = 0; h < H; h++) {
        const i64 o = h * 3 * HS;
        i64 q[64], k[64], q16[64];
        memcpy(q, qkv + o, sizeof(i64) * HS);
        memcpy(k, qkv + o + HS, sizeof(i64) * HS);
        pturn(M, q, p, st);
        pturn(M, k, p, st);
        const i64 eq = orc_to16_row(q, HS, -16, q16);
        EK[p * H + h] = orc_to16_row(k, HS, -16, K16 + p * d + h * HS);
        memcpy(V + p * d + h * HS, qkv + o + 2 * HS, sizeof(i64) * HS);
        for (i64 s = 0; s <= p; s++) {
            i64 dot = 0;
            for (i64 t = 0; t < HS; t++) dot += q16[t] * K16[s * d + h * HS + t];
            sc[s] = ppow(dot, wsub(wmul(eq + EK[s * H + h] + 10, 65536), M->half), M->exp2t, st);
        }
        const i64 lev = sc[orc_race(sc, p + 1)];
        i64 Z = 0, vmax = 0, num[64] = {0};
        for (i64 s = 0; s <= p; s++)
            for (i64 t = 0; t < HS; t++) { const i64 av = iabs(V[s * d + h * HS + t]); if (av > vmax) vmax = av; }
        for (i64 s = 0; s <= p; s++) {
            const i64 dd = wsub(lev, sc[s]);
            const i64 a = dd < M->alen ? M->arr[dd] : 0;
            if (!a) continue;
            Z += a;
            for (i64 t = 0; t < HS; t++) num[t] = wadd(num[t], wmul(a, V[s * d + h * HS + t]));
        }
        if ((double)vmax * (double)Z >= 4611686018427387904.0) flag(st, PYO_E_ATT);
        const i64 F = -orc_log2fix1(Z, M->log2t);
        for (i64 t = 0; t < HS; t++) out[h * HS + t] = ppow(num[t], F, M->exp2t, st);
    }
}

static double plate_max(const int16_t* w, i64 n) {
    int m = 0;
    for (i64 i = 0; i < n; i++) { int a = w[i] < 0 ? -w[i] : w[i]; if (a > m) m = a; }
    return (double)m;
}

/* the largest |w| of every plate (product's assert, pythia_base2.py:75) */
void pyo_prepare(py_model* M) {
    for (i64 l = 0; l < M->L; l++)
        for (int k = 0; k < 4; k++) M->wmax[l][k] = plate_max(M->w[l][k], (i64)PNIN[k] * PNOUT[k]);
    M->hwmax = plate_max(M->hw, M->d * M->vocab);
}

/* ---------------- KV-cached machine ---------------- */
typedef struct {
    int64_t max_ctx, pos;
    int64_t* K16; int64_t* EK; int64_t* V;   /* [L][ctx][768], [L][ctx][heads], [L][ctx][768] */
    int64_t* R;                               /* [768] */
} py_kv;

py_kv* pyo_kv_new(const py_model* M, int64_t max_ctx) {
    py_kv* S = calloc(1, sizeof(py_kv));
    S->max_ctx = max_ctx;
    S->K16 = calloc((size_t)M->L * max_ctx * M->d, sizeof(i64));
    S->EK = calloc((size_t)M->L * max_ctx * M->heads, sizeof(i64));
    S->V = calloc((size_t)M->L * max_ctx * M->d, sizeof(i64));
    S->R = calloc((size_t)M->d, sizeof(i64));
    return S;
}
void pyo_kv_free(py_kv* S) { if (!S) return; free(S->K16); free(S->EK); free(S->V); free(S->R); free(S); }

#define PX(p, l, k) ((p) + ((l) * 4 + (k)) * 3072)

/* one new position: word `tok` enters at S->pos; returns the next word when want_head, else -1 */
int64_t pyo_step(const py_model* M, py_kv* S, int32_t tok, int want_head, py_rec* rec, int* status) {
    int st = 0;
    if (S->pos >= S->max_ctx || S->pos >= M->npos || tok < 0 || tok >= M->vocab) { *status = ORC_E_ARG; return -1; }
    const i64 d = M->d, p = S->pos;
    i64* R = S->R;
    i64 g[768], qkv[2304], att[768], fcv[3072], hid[3072], At[768], Mo[768], x16[3072], pile[3072];
    i64* sc = malloc(sizeof(i64) * (p + 1));
    for (i64 i = 0; i < d; i++) R[i] = prsh((i64)M->ew[(i64)tok * d + i], -(M->ee[tok] + 16), &st);
    for (i64 l = 0; l < M->L; l++) {
        i64 ex;
        if (rec && rec->stream) memcpy(rec->stream + l * 768, R, sizeof(i64) * 768);
        pgauge(M, R, M->ng[l][0], M->nge[l][0], M->nb[l][0], g, &st);
        if (rec && rec->g1) memcpy(rec->g1 + l * 768, g, sizeof(i64) * 768);
#define KEEP(k, n_in, n_out, outv)                                                               \
        if (rec) {                                                                                \
            if (rec->x16) memcpy(PX(rec->x16, l, k), x16, sizeof(i64) * (n_in));                  \
            if (rec->ex) rec->ex[l * 4 + (k)] = ex;                                               \
            if (rec->pile) memcpy(PX(rec->pile, l, k), pile, sizeof(i64) * (n_out));              \
            if (rec->out) memcpy(PX(rec->out, l, k), outv, sizeof(i64) * (n_out));                \
        }
        ex = pplain(M->w[l][0], M->e[l][0], M->b[l][0], M->wmax[l][0], g, 768, 2304, qkv, x16, pile, &st);
        KEEP(0, 768, 2304, qkv)
        pattend(M, qkv, p, S->K16 + (size_t)l * S->max_ctx * d, S->EK + (size_t)l * S->max_ctx * M->heads,
                S->V + (size_t)l * S->max_ctx * d, sc, att, &st);
        if (rec && rec->att) memcpy(rec->att + l * 768, att, sizeof(i64) * 768);
        ex = pplain(M->w[l][1], M->e[l][1], M->b[l][1], M->wmax[l][1], att, 768, 768, At, x16, pile, &st);
        KEEP(1, 768, 768, At)
        pgauge(M, R, M->ng[l][1], M->nge[l][1], M->nb[l][1], g, &st);
        if (rec && rec->g2) memcpy(rec->g2 + l * 768, g, sizeof(i64) * 768);
        ex = pplain(M->w[l][2], M->e[l][2], M->b[l][2], M->wmax[l][2], g, 768, 3072, fcv, x16, pile, &st);
        KEEP(2, 768, 3072, fcv)
        for (int j = 0; j < 3072; j++) hid[j] = orc_edge1(fcv[j], M->phi);
        if (rec && rec->hid) memcpy(rec->hid + l * 3072, hid, sizeof(i64) * 3072);
        ex = pplain(M->w[l][3], M->e[l][3], M->b[l][3], M->wmax[l][3], hid, 3072, 768, Mo, x16, pile, &st);
        KEEP(3, 3072, 768, Mo)
#undef KEEP
        for (i64 i = 0; i < d; i++) R[i] = wadd(wadd(R[i], At[i]), Mo[i]);
    }
    free(sc);
    S->pos++;
    i64 word = -1;
    if (want_head) {
        if (rec && rec->stream_final) memcpy(rec->stream_final, R, sizeof(i64) * 768);
        pgauge(M, R, M->fg, M->fge, M->fb, g, &st);
        if (rec && rec->glnf) memcpy(rec->glnf, g, sizeof(i64) * 768);
        i64* hp = malloc(sizeof(i64) * M->vocab);
        i64* lg = malloc(sizeof(i64) * M->vocab);
        const i64 ey = pplain(M->hw, M->he, NULL, M->hwmax, g, 768, M->vocab, lg, x16, hp, &st);
        word = orc_race(lg, M->vocab);
        if (rec) {
            if (rec->hx16) memcpy(rec->hx16, x16, sizeof(i64) * 768);
            if (rec->hex) *rec->hex = ey;
            if (rec->hpile) memcpy(rec->hpile, hp, sizeof(i64) * M->vocab);
            if (rec->logits) memcpy(rec->logits, lg, sizeof(i64) * M->vocab);
        }
        free(hp); free(lg);
    }
    *status = st;
    return word;
}

void pyo_read_kv(const py_model* M, const py_kv* S, int64_t l, int64_t p, int64_t* k16, int64_t* ek, int64_t* v) {
    const size_t base = ((size_t)l * S->max_ctx + p);
    memcpy(k16, S->K16 + base * M->d, sizeof(i64) * M->d);
    memcpy(ek, S->EK + base * M->heads, sizeof(i64) * M->heads);
    memcpy(v, S->V + base * M->d, sizeof(i64) * M->d);
}
void pyo_resid(const py_model* M, const py_kv* S, int64_t* out) { memcpy(out, S->R, sizeof(i64) * M->d); }

/* pythia_base2.py:125-141 on a whole QKV matrix [P][3d] (positions 0..P-1) -> out [P][d] */
int pyo_attention(const py_model* M, const int64_t* QKV, int64_t P, int64_t* out) {
    int st = 0;
    const i64 d = M->d;
    i64* K16 = calloc((size_t)P * d, sizeof(i64));
    i64* EK = calloc((size_t)P * M->heads, sizeof(i64));
    i64* V = calloc((size_t)P * d, sizeof(i64));
    i64* sc = malloc(sizeof(i64) * P);
    for (i64 p = 0; p < P; p++) pattend(M, QKV + p * 3 * d, p, K16, EK, V, sc, out + p * d, &st);
    free(K16); free(EK); free(V); free(sc);
    return st;
}
