// gfx950 kernels of the integer GPT-2 decode step (one new position per stream).
//
// The weight product (base2.py:29-32) is a wave-cooperative GEMV over a column-tiled int16 plate:
//   * the plate is cut into tiles of TC output columns; inside a tile the 16-byte unit u holds 8 consecutive
//     inputs (k = 8 (u / TC) .. + 8) of column u % TC, so one 256-thread block streams a tile as perfectly
//     contiguous 16-byte loads;
//   * the light x16 (17-bit, [-32768, 32768]) is split once per phase into xh = x >> 8 in [-128, 128] and
//     xl = x & 255, kept in LDS as packed int16 pairs; each 16-byte weight load then feeds 8 v_dot2_i32_i16
//     (sdot2) instructions: ah += w . xh, al += w . xl.  Every partial term is below 2^24 and a thread sums at
//     most 96 of them, so the 32-bit cells never carry; the pile is formed once in 64 bits as ah * 256 + al.
//     That is the reference's "two narrow cells combined once at the end" (SPEC.md:28, fr2 gatew) with the
//     split taken on the light instead of on the product; the pile is the same exact integer.
//   * the phase's whole-row dependencies (the water level's OR, the gauge's S1 and S2) are recomputed by every
//     block from the row in L2 (768 or 3072 values) so that prologue, product and epilogue fuse into one
//     launch and the next phase needs no extra pass.
//   * a phase's critical path holds one dependent memory read (the row it consumes): the weights, exponents
//     and biases of the block's first tile are requested before it, the gauge's power factor EXP2[f] is one
//     value per block (f = -LS mod 2^16 for every column),.
#include "sm_kernels.h"

// The float stages below evaluate each float64 operation of the reference's expression on its own, rounded once
// in numpy's order: no multiply and add are fused into one rounding anywhere in this library.
#pragma clang fp contract(off)

#define NTHR 256

// ---------------------------------------------------------------------------------------------------------
// block reductions (NW waves, 4 by default).  red: NW slots, free on entry; every thread gets the result.
template <typename F, int NW = 4>
SMD i64 block_reduce(i64 v, i64* red, F op, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    v = wave_reduce64(v, op);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    i64 r = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) r = op(r, red[w]);
    __syncthreads();
    return r;
}
// two sums in one pass
SMD void block_sum2(i64& a, i64& b, i64* red, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { a += __shfl_xor(a, o, 64); b += __shfl_xor(b, o, 64); }
    if (lane == 0) { red[wave] = a; red[4 + wave] = b; }
    __syncthreads();
    a = red[0] + red[1] + red[2] + red[3];
    b = red[4] + red[5] + red[6] + red[7];
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------
// The float stages (base2.py:10-11 gauge=/edge=; foundation0/pythia_base2.py:21-27): diagnostics that put one
// stage back to float64.
//
// numpy's sum of 768 float64 values (its pairwise summation): halves at multiples of 8 down to blocks of 96, each
// block summed by 8 strided accumulators that are combined as ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)).
// One wave: lane l runs accumulator l % 8 of block l / 8; the butterfly over lane bits 0-2, then 3-5, forms the
// same tree (a + b == b + a exactly), and every lane ends with the total.  val(i) gives element i.
template <typename F>
SMD double np_sum768(F val, int lane) {
    const int base = 96 * (lane >> 3) + (lane & 7);
    double r = val(base);
#pragma unroll
    for (int t = 1; t < 12; t++) r += val(base + 8 * t);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) r += __shfl_xor(r, o, 64);
    return r;
}
// the float gauge's size of a 768-wide row held as float64 in LDS: mean, then sqrt(mean((x - mean)^2) + 1e-5)
// (base2.py:67, 111; foundation0/pythia_base2.py:103); the mean returned in mu
SMD double np_sigma768(const double* xf, int lane, double& mu) {
    const double m = np_sum768([&](int i) { return xf[i]; }, lane) / 768.0;
    const double v = np_sum768([&](int i) { const double d = xf[i] - m; return d * d; }, lane) / 768.0;
    mu = m;
    return sqrt(v + 1e-5);
}
// edge=float, GPT-2 (base2.py:80): round(0.5 h (1 + tanh(0.7978845608028654 (h + 0.044715 h^3))) 2^16), h = H 2^-16
SMD i64 edge_tanh(i64 H) {
    const double h = (double)H * (1.0 / 65536.0);
    const double u = 0.7978845608028654 * (h + 0.044715 * pow(h, 3.0));
    return (i64)rint(0.5 * h * (1.0 + tanh(u)) * 65536.0);
}
// edge=float, Pythia (foundation0/pythia_base2.py:144-146): round(h 0.5 (1 + erf(h / sqrt(2))) 2^16)
SMD i64 edge_erf(i64 H) {
    const double h = (double)H * (1.0 / 65536.0);
    return (i64)rint(h * 0.5 * (1.0 + erf(h / 1.4142135623730951)) * 65536.0);
}

// ---------------------------------------------------------------------------------------------------------
// Prologue: the light entering the plate, computed by every block from the row it reads (NIN values over the
// block's NT threads).  Writes xh/xl (NIN shorts each) into LDS and returns ex, LS and the gauge's power factor.
// The water level's OR is reduced as two 32-bit words and the gauge's sums as exact 32-bit pieces (S1 < 2^25,
// S2 split at bit 16), each wave through DPP and the waves through one LDS exchange.
// the row's loads, issued first: vector loads complete in order, so anything requested before them (plate
// tiles from HBM) would have to arrive before the row could be used
template <int NIN, int NT, int PRO>
SMD void prologue_load(const GemvArgs& a, int tid, i64 (&v)[NIN / NT], int (&gq)[NIN / NT], i64 (&bq)[NIN / NT]) {
    constexpr int PER = NIN / NT;
    if constexpr (PRO == PRO_RACE) {
        // the step before's head bests (two a thread; bounded loads, a best past the last block reads as none),
        // then its position and the next position's row of wpe; the word's wte row follows the race (race_row)
        static_assert(NIN == 768 && NT == 256, "layer 0's qkv: 768 inputs over 256 threads");
        const Race1Args& r = a.race;
        const __amdgpu_buffer_rsrc_t rv = buf_rsrc(r.part_v, (unsigned)r.nblk * 8u), ri = buf_rsrc(r.part_i, (unsigned)r.nblk * 4u);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int g = tid + 256 * k;
            bq[k] = buf_load8(rv, (unsigned)g * 8u);
            const int i = buf_load1(ri, (unsigned)g * 4u);
            gq[k] = g < r.nblk ? i : -1;
        }
        const int q = *r.pos + 1;                       // (no row of wpe past its last position: zeros)
        const __amdgpu_buffer_rsrc_t rp = buf_rsrc(r.wpe + (size_t)(q < r.npos ? q : 0) * 768, q < r.npos ? 768u * 8u : 0u);
#pragma unroll
        for (int m = 0; m < PER; m++) v[m] = buf_load8(rp, (unsigned)(tid + NT * m) * 8u);
        return;
    }
    if constexpr (PRO == PRO_ATT || PRO == PRO_PATT) {
        // element 64 h + d: head h's value sum d; thread t < 12 also head t's arrival sum (bq[0]) and largest
        // weighed |v| (bq[1]); bounded loads, no branch
        static_assert(NIN == 768 && PER >= 2, "the attention row is 768 wide");
#pragma unroll
        for (int m = 0; m < PER; m++) {
            const int i = tid + NT * m;
            v[m] = a.aacc[(i >> 6) * 68 + (i & 63)];
        }
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a.aacc, 12u * 68u * 8u);
        bq[0] = buf_load8(ra, (unsigned)(tid * 68 + 64) * 8u);
        bq[1] = buf_load8(ra, (unsigned)(tid * 68 + 65) * 8u);
        return;
    }
#pragma unroll
    for (int m = 0; m < PER; m++) v[m] = a.X[tid + NT * m];
    if (PRO == PRO_PGAUGE) {
#pragma unroll
        for (int m = 0; m < PER; m++) { gq[m] = a.ng[tid + NT * m]; bq[m] = a.nb[tid + NT * m]; }
    }
}

// Pythia's prologue (foundation0/pythia_base2.py:100-110, 113): the gauge of the stream row R with the norm's own
// gain and offset, then that row's water level.  Three block reductions: R's OR, the sums S1, S2, the gauged
// row's OR.  c g < 2^41 and EXP2 < 2^17, so c g EXP2[f] is exact in 64 bits as the reference's int64 path is.
// FG (gauge=float, :102-104): round((x - mu) / sigma g 2^ge 2^16) + b with x = R 2^-16 in float64 (xf: 768 doubles
// of LDS), in place of the first two reductions.
template <int NT, int FG>
SMD void prologue_py(const GemvArgs& a, int tid, const i64 (&v)[768 / NT], const int (&gq)[768 / NT],
                     const i64 (&bq)[768 / NT], short* xh_s, short* xl_s, int* red, double* xf, i64& ex_o, bool rec) {
    constexpr int PER = 768 / NT, NW = NT / 64;
    const int lane = tid & 63, wave = tid >> 6;
    i64 g[PER];
    if constexpr (FG) {
#pragma unroll
        for (int m = 0; m < PER; m++) xf[tid + NT * m] = (double)v[m] * (1.0 / 65536.0);
        __syncthreads();
        double mu;
        const double sg = np_sigma768(xf, lane, mu), sc = ldexp(1.0, a.nge + 16);
#pragma unroll
        for (int m = 0; m < PER; m++) {
            const double d = xf[tid + NT * m] - mu;
            g[m] = wadd((i64)rint(d / sg * (double)gq[m] * sc), bq[m]);
            if (rec && a.rg) a.rg[tid + NT * m] = g[m];
        }
    } else {
        u64 o = 0;
#pragma unroll
        for (int m = 0; m < PER; m++) o |= (u64)iabs64(v[m]);
        unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
        if (lane == 0) { red[2 * wave] = (int)olo; red[2 * wave + 1] = (int)ohi; }
        __syncthreads();
        u64 all = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) all |= ((u64)(unsigned)red[2 * w + 1] << 32) | (unsigned)red[2 * w];
        const int sh = water_shift((i64)all);
        int xi[PER];
        int s1 = 0;
        i64 s2 = 0;
#pragma unroll
        for (int m = 0; m < PER; m++) {
            xi[m] = (int)rsh(v[m], sh);
            s1 += xi[m];
            s2 += (i64)xi[m] * xi[m];
        }
        const int w1 = wave_add32(s1), w2h = wave_add32((int)(s2 >> 16)), w2l = wave_add32((int)(s2 & 0xFFFF));
        if (lane == 0) { red[32 + 3 * wave] = w1; red[33 + 3 * wave] = w2h; red[34 + 3 * wave] = w2l; }
        __syncthreads();
        i64 S1 = 0, S2h = 0, S2l = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) { S1 += red[32 + 3 * w]; S2h += red[33 + 3 * w]; S2l += red[34 + 3 * w]; }
        i64 e2;
        const i64 ls = pgauge_ls_pow(S1, (S2h << 16) + S2l, -16 + sh, a.tb, e2);
        const i64 sg = wsub(16, wsub(wmul((i64)a.nge + 16, 65536), ls) >> 16);     // 16 - I of the gauge's power
#pragma unroll
        for (int m = 0; m < PER; m++) {
            const i64 c = 768 * (i64)xi[m] - S1;
            g[m] = wadd(rsh(wmul(c * gq[m], e2), sg), bq[m]);
            if (rec && a.rg) a.rg[tid + NT * m] = g[m];
        }
    }
    u64 o = 0;
#pragma unroll
    for (int m = 0; m < PER; m++) o |= (u64)iabs64(g[m]);
    unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
    if (lane == 0) { red[72 + 2 * wave] = (int)olo; red[73 + 2 * wave] = (int)ohi; }
    __syncthreads();
    u64 all = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) all |= ((u64)(unsigned)red[73 + 2 * w] << 32) | (unsigned)red[72 + 2 * w];
    const int sh2 = water_shift((i64)all);
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + NT * m;
        const int x16 = (int)rsh(g[m], sh2);
        xh_s[i] = (short)(x16 >> 8);
        xl_s[i] = (short)(x16 & 255);
        if (rec && a.rx16) a.rx16[i] = x16;
    }
    if (rec && a.rexls && tid == 0) { a.rexls[0] = -16 + sh2; a.rexls[1] = 0; }
    ex_o = -16 + sh2;
    __syncthreads();
}
// MODE_INV (the complement machine): a PRO_GAUGE row is the stream, held complemented, and is read back plain; the
// light is held complemented in LDS, and sx_o returns the plain light's sum (the pile's correction).
// MODE_FGAUGE with PRO_GAUGE (gauge=float, base2.py:67): sig_o = the row's float64 size (xf: 768 doubles of LDS).
// TOP (the top read's first stage): the light held in LDS as (x0, x2), (x1, x3) of every group of four inputs (the
// high-byte plane's pairs), nn_o = the sum of its negative values; block 0 writes the light and its facts.
template <int NIN, int NT, int PRO, int MODE, bool TOP = false>
SMD void prologue(const GemvArgs& a, int tid, const i64 (&vin)[NIN / NT], short* xh_s, short* xl_s, int* red,
                  double* xf, i64& ex_o, i64& ls_o, i64& e2_o, i64& sx_o, double& sig_o, i64& nn_o, bool rec) {
    constexpr int PER = NIN / NT, NW = NT / 64;
    constexpr bool INV = MODE & MODE_INV, FG = (MODE & MODE_FGAUGE) && PRO == PRO_GAUGE;
    static_assert(!TOP || (PRO == PRO_GAUGE && NW <= 8 && !INV), "the top read lights the stream row");
    static_assert(!FG || NIN == 768, "the float gauge reads a 768-wide stream row");
    const int lane = tid & 63, wave = tid >> 6;
    i64 v[PER];
#pragma unroll
    for (int m = 0; m < PER; m++) v[m] = INV && PRO == PRO_GAUGE ? ~vin[m] : vin[m];
    if constexpr (FG) {
#pragma unroll
        for (int m = 0; m < PER; m++) xf[tid + NT * m] = (double)v[m] * (1.0 / 65536.0);   // (the next barrier serves)
    }
    int sh = 0;
    if (PRO != PRO_X16) {
        u64 o = 0;
#pragma unroll
        for (int m = 0; m < PER; m++) o |= (u64)iabs64(v[m]);
        const unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
        if (lane == 0) { red[2 * wave] = (int)olo; red[2 * wave + 1] = (int)ohi; }
        __syncthreads();
        u64 all = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) all |= ((u64)(unsigned)red[2 * w + 1] << 32) | (unsigned)red[2 * w];
        sh = water_shift((i64)all);
    }
    if constexpr (FG) {
        double mu;
        sig_o = np_sigma768(xf, lane, mu);
    }
    const i64 ex = -16 + sh;
    int s1 = 0, sn = 0;
    i64 s2 = 0;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        int i = tid + NT * m;
        const int xi = PRO == PRO_X16 ? (int)v[m] : (int)rsh(v[m], sh);
        const int xs = INV ? ~xi : xi;          // the light as held
        const int li = TOP ? (i & ~3) | ((i & 1) << 1) | ((i >> 1) & 1) : i;
        xh_s[li] = (short)(xs >> 8);            // in [-129, 128]
        xl_s[li] = (short)(xs & 255);
        s1 += xi;
        s2 += (i64)xi * xi;
        if (TOP) sn += min(xi, 0);
        if (rec && a.rx16) a.rx16[i] = xi;
        if (TOP && blockIdx.x == 0) a.tx[i] = xi;
    }
    i64 ls = 0, e2 = 0;
    if (PRO == PRO_GAUGE) {
        const int w1 = wave_add32(s1), w2h = wave_add32((int)(s2 >> 16)), w2l = wave_add32((int)(s2 & 0xFFFF));
        if (lane == 0) { red[32 + 3 * wave] = w1; red[33 + 3 * wave] = w2h; red[34 + 3 * wave] = w2l; }
        if constexpr (TOP) {
            const int wn = wave_add32(sn);
            if (lane == 0) red[80 + wave] = wn;
        }
        __syncthreads();
        i64 S1 = 0, S2h = 0, S2l = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) { S1 += red[32 + 3 * w]; S2h += red[33 + 3 * w]; S2l += red[34 + 3 * w]; }
        ls = gauge_ls_pow<true>(S1, (S2h << 16) + S2l, ex, a.tb, e2);
        sx_o = S1;
        if constexpr (TOP) {
            i64 nn = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) nn += red[80 + w];
            nn_o = nn;
            if (blockIdx.x == 0 && tid == 0) { a.tf[0] = ex; a.tf[1] = ls; a.tf[2] = e2; }
        }
    } else if (INV) {
        const int w1 = wave_add32(s1);
        if (lane == 0) red[32 + wave] = w1;
        __syncthreads();
        i64 S1 = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) S1 += red[32 + w];
        sx_o = S1;
    } else {
        __syncthreads();
    }
    if (rec && a.rexls && tid == 0) { a.rexls[0] = ex; a.rexls[1] = ls; }
    ex_o = ex;
    ls_o = ls;
    e2_o = e2;
}

// PRO_RACE: the race over the step before's head bests (race1_finish's arithmetic, in every block), the word fed
// back: v[m] turns from the next position's wpe row into the entering row wte[word] + wpe[q] (base2.py:103).
// A prompt position's next word is the prompt's.  Block 0 writes the word, the counters, the next position slot
// and the row (proj's layer-0 addition reads it).  pv, pi: the thread's two bests; bvs, bis: a slot a wave.
template <int NT>
SMD void race_row(const GemvArgs& a, int tid, i64 (&v)[768 / NT], const i64 (&pv)[768 / NT], const int (&pi)[768 / NT],
                  i64* bvs, int* bis, int* tok_s) {
    constexpr int PER = 768 / NT, NW = NT / 64;
    const Race1Args& r = a.race;
    const int lane = tid & 63, wave = tid >> 6;
    i64 bv = 0;
    int bi = -1;
#pragma unroll
    for (int k = 0; k < 2; k++)
        if (race_beats<0>(pv[k], pi[k], bv, bi)) { bv = pv[k]; bi = pi[k]; }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const i64 ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (race_beats<0>(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { bvs[wave] = bv; bis[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        bv = bvs[0]; bi = bis[0];
        for (int w = 1; w < NW; w++)
            if (race_beats<0>(bvs[w], bis[w], bv, bi)) { bv = bvs[w]; bi = bis[w]; }
        const int p = *r.pos, plen = *r.plen, q = p + 1;
        const bool known = p < plen - 1;                // a prompt position: the next word is the prompt's
        const int tok = known ? r.seq[q] : bi;
        if (blockIdx.x == 0) {
            if (!known) {
                r.seq[q] = bi;
                r.words[q - plen] = bi;
            }
            *r.nwords = q - plen + 1;
            *r.pos_next = q;
        }
        *tok_s = tok;
    }
    __syncthreads();
    const size_t tok = (size_t)*tok_s;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + NT * m;
        v[m] = wadd(r.wte[tok * 768 + i], v[m]);
        if (blockIdx.x == 0) r.R0[i] = v[m];
    }
}

// PRO_ATT / PRO_PATT: the attention row from the heads' accumulators, k_att_finish's arithmetic in every block
// (base2.py:99; pythia_base2.py:139, 90).  Thread t < 12 forms head t's divisor, -log2fix(Z) and its power
// factor (one gather of the two table entries for the twelve heads), into fz; after one barrier v[m] turns from
// head h's value sum into its output.  zq: thread t < 12's arrival sum and largest weighed |v|.  Block 0 raises
// the Pythia asserts and writes the record.
template <int NT, bool PY>
SMD void att_row(const GemvArgs& a, int tid, i64 (&v)[768 / NT], const i64 (&zq)[768 / NT], int* fz, bool rec) {
    constexpr int PER = 768 / NT;
    if (tid < 12) {
        int zt;
        i64 zm;
        log2_parts(zq[0], zt, zm);
        fz[2 * tid] = -(zt * 65536 + (int)tab_log2(a.tb, zm));          // -log2fix(Z): |.| < 2^23
        fz[2 * tid + 1] = (int)tab_hpow(a.tb, zm);
        if (PY && blockIdx.x == 0 && a.err && (double)zq[1] * (double)zq[0] >= 4611686018427387904.0)
            atomicOr(a.err, SM_ERR_RANGE);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int i = tid + NT * m, h = i >> 6;
        const i64 F = fz[2 * h], zhp = fz[2 * h + 1];
        i64 o;
        if constexpr (PY) {
            const __int128 X = (__int128)v[m] * zhp;
            const i64 sft = 16 - (F >> 16);
            const __int128 r = sft >= 100 ? (__int128)0 : (X + ((__int128)1 << (sft - 1))) >> sft;
            if (blockIdx.x == 0 && a.err && (r > (__int128)INT64_MAX || r < (__int128)INT64_MIN)) atomicOr(a.err, SM_ERR_RANGE);
            o = (i64)r;
        } else {
            o = power_e(v[m], F, F & 0xFFFF, zhp, a.tb);
        }
        v[m] = o;
        if (rec && blockIdx.x == 0 && a.ratt) a.ratt[i] = o;
    }
}

// ---------------------------------------------------------------------------------------------------------
// One wave's share of a tile: U units of 16 bytes per lane (unit u = lane + 64 m).  WB: bytes a weight (2: the
// int16 plate; 1: the top read's high-byte plane, w >> 8)
template <int NIN, int TC, int WB = 2>
struct WaveTile {
    static constexpr int U = TC * NIN * WB / 16 / 64;
    static_assert(TC * NIN * WB / 16 % 64 == 0, "a tile must split evenly over the 64 lanes");
};

template <int NIN, int TC, int U, int WB = 2>
SMD void load_wtile(v4i (&w)[U], const int4* __restrict__ W, int tile, int lane) {
    const v4i* base = reinterpret_cast<const v4i*>(W) + (size_t)tile * (TC * NIN * WB / 16) + lane;
#pragma unroll
    for (int m = 0; m < U; m++) w[m] = base[64 * m];      // plain loads: measured 1 % faster a step than nontemporal
}

// the lane's part of its column's pile: unit u holds inputs 8 (u / TC) .. + 8 of column u % TC = lane % TC
// (WB = 1: inputs 16 (u / TC) .. + 16, as signed bytes)
template <int NIN, int TC, int U, int WB = 2>
SMD i64 wtile_partial(const v4i (&w)[U], const short* xh_s, const short* xl_s, int lane) {
    int ah = 0, al = 0;
#pragma unroll
    for (int m = 0; m < U; m++) {
        const int c = (lane + 64 * m) / TC;
        const v4i ww = w[m];
        if constexpr (WB == 2) {
            const int4 xh = reinterpret_cast<const int4*>(xh_s)[c];
            const int4 xl = reinterpret_cast<const int4*>(xl_s)[c];
            ah = dot2(ww.x, xh.x, ah); ah = dot2(ww.y, xh.y, ah); ah = dot2(ww.z, xh.z, ah); ah = dot2(ww.w, xh.w, ah);
            al = dot2(ww.x, xl.x, al); al = dot2(ww.y, xl.y, al); al = dot2(ww.z, xl.z, al); al = dot2(ww.w, xl.w, al);
        } else {
            // dword d holds the bytes of inputs 4d .. 4d + 3; (d << 8) & 0xFF00FF00 and d & 0xFF00FF00 are the
            // int16 pairs (256 b0, 256 b2) and (256 b1, 256 b3): the high byte's share of the pile with its 256
            // already in place; the light is held in LDS as (x0, x2), (x1, x3) of every group of four
            const int4 h0 = reinterpret_cast<const int4*>(xh_s)[2 * c], h1 = reinterpret_cast<const int4*>(xh_s)[2 * c + 1];
            const int4 l0 = reinterpret_cast<const int4*>(xl_s)[2 * c], l1 = reinterpret_cast<const int4*>(xl_s)[2 * c + 1];
            const int hx[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            const int lx[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const int wd[4] = {ww.x, ww.y, ww.z, ww.w};
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const int pa = (int)(((unsigned)wd[d] << 8) & 0xFF00FF00u), pb = (int)((unsigned)wd[d] & 0xFF00FF00u);
                ah = dot2(pa, hx[2 * d], ah); ah = dot2(pb, hx[2 * d + 1], ah);
                al = dot2(pa, lx[2 * d], al); al = dot2(pb, lx[2 * d + 1], al);
            }
        }
    }
    return (i64)ah * 256 + (i64)al;
}

// The phase kernel.  NT = 64 WPB threads; every wave owns whole tiles (wave-global index w, tiles w, w + G, ..),
// so after the block's prologue no block barrier is needed: a wave loads its tile, forms its TC piles with DPP
// steps, and lanes 16 - TC .. 15 apply the epilogue of one column each.  The next tile of the wave (if any)
// is in flight while the current one is reduced.
// The first memory requests are the row and the first tile: nothing the kernel reads depends on another read
// (the position is not needed; REC = 1 instantiations, launched only for a recorded step, compare it).
// MODE (batch 1): MODE_INV, the complement machine (GPT-2's phases; see race_beats; recorded values are the plain
// machine's); MODE_FGAUGE, MODE_FEDGE: the float gauge (gauged phases) and the float edge (the fc phases).
template <int NIN, int TC, int WPB, int PRO, int EPI, int REC, int MODE = 0>
__global__ __launch_bounds__(64 * WPB) void k_gemv(GemvArgs a) {
    constexpr bool INV = MODE & MODE_INV;
    constexpr bool FG = (MODE & MODE_FGAUGE) && (PRO == PRO_GAUGE || PRO == PRO_PGAUGE);
    constexpr bool FE = (MODE & MODE_FEDGE) && (EPI == EPI_GAUGED_EDGE || EPI == EPI_PLAIN_EDGE);
    static_assert(!INV || PRO == PRO_GAUGE || PRO == PRO_TO16 || PRO == PRO_ATT, "the complement machine is GPT-2's");
    constexpr bool TOP = EPI == EPI_TOP1;
    constexpr bool SPLIT = MODE & MODE_SPLIT;
    static_assert(!SPLIT || (!TOP && !INV), "split plates are the Pythia machine's");
    constexpr int WB = TOP ? 1 : 2;                   // the top read's first stage streams the high-byte plane
    constexpr int NT = 64 * WPB, U = WaveTile<NIN, TC, WB>::U, U2 = SPLIT ? U : 1;
    static_assert(NIN % NT == 0, "the block's threads must split the light row evenly");
    __shared__ __align__(16) short xh_s[NIN];
    __shared__ __align__(16) short xl_s[NIN];
    __shared__ double xf_s[FG ? 768 : 1];
    __shared__ int red[96];        // prologue: OR words [0, 24), sums [32, 68), second OR [72, 96)
    __shared__ int fz[PRO == PRO_ATT || PRO == PRO_PATT ? 24 : 1];   // the heads' divisors (att_row)
    __shared__ int race_tok;                                         // PRO_RACE: the word fed back
    __shared__ i64 bestv[WPB];
    __shared__ int besti[WPB];
    // EPI_TOP1: each finished word of the block (slot (wave, tile of the wave, column)): word, high bound, coarse pile
    constexpr int TSLOTS = TOP ? WPB * TOP_ITERS * TC : 1;
    __shared__ int top_j[TSLOTS];
    __shared__ i64 top_h[TSLOTS], top_c[TSLOTS];
    __shared__ int top_n;
    static_assert(WPB <= 12, "the prologue's LDS slots hold at most 12 waves");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane - (16 - TC);                 // the column this lane finishes (valid when 0 <= col < TC)
    const bool fin = col >= 0 && col < TC;
    constexpr bool HEAD = EPI == EPI_HEAD || EPI == EPI_PHEAD;
    if constexpr (TOP) {                              // (the prologue's barriers come before any slot is written)
        for (int k = tid; k < TSLOTS; k += NT) top_j[k] = -1;
        if (tid == 0) top_n = 0;
    }

    i64 best_v = TOP ? INT64_MIN : 0;                 // EPI_TOP1: the lane's best low
    int best_i = -1;
    {
        const int gw = blockIdx.x * WPB + wave, nw = gridDim.x * WPB;
        // two named buffers in turn (no register copies, so a prefetch in flight is never waited on early);
        // a tile's exponents and biases are requested before its weights, so waiting for the small loads
        // never waits for the large ones behind them
        v4i wA[U], wB[U], wA2[U2], wB2[U2];          // (wA2, wB2: MODE_SPLIT's subtracted plate)
        i64 bA = 0, eA = 0, bB = 0, eB = 0, sA = 0, sB = 0;     // (EPI_PLAIN_ADD: sA, sB hold the row added to)
        // every lane loads (indices clamped into range): a load that writes only some lanes would have to be
        // merged with the register's old value, and that merge waits for the load
        auto fetch = [&](v4i (&w)[U], v4i (&w2)[U2], i64& we_, i64& b_, i64& s_, int t) {
            t = t < a.ntiles ? t : a.ntiles - 1;
            if (EPI != EPI_PILE) {
                int j = t * TC + col;
                j = j < 0 ? 0 : (j < a.nout ? j : a.nout - 1);
                we_ = a.we[j];
                if (EPI != EPI_PHEAD) b_ = a.bias[j];
                if (INV) s_ = a.sw[j];
                else if (EPI == EPI_PLAIN_ADD) s_ = a.Yb[j];
            }
            load_wtile<NIN, TC, U, WB>(w, a.W, t, lane);
            if constexpr (SPLIT) load_wtile<NIN, TC, U, WB>(w2, a.W2, t, lane);
        };
        int tile = gw;
        i64 row[NIN / NT], nbq[NIN / NT];
        int ngq[NIN / NT];
        prologue_load<NIN, NT, PRO>(a, tid, row, ngq, nbq);   // the row first, then this wave's first tile
        fetch(wA, wA2, eA, bA, sA, tile);               // unconditional (clamped): no branch for the wait count to merge
        // then the next phase's lines (a fixed count a thread, clamped to a valid address: no branch around loads);
        // their values are consumed only after the tiles, where they have long arrived
        int pfs = 0;
        {
            constexpr int PFN = WPB <= 2 ? 2 : 1;
            const char* pb = a.pf ? a.pf : reinterpret_cast<const char*>(a.W);
            const int lines = a.pf ? a.pf_lines : 1;
#pragma unroll
            for (int k = 0; k < PFN; k++) {
                const int i = tid + NT * k, r = i / lines, l = i - r * lines;
                const int b2 = blockIdx.x + r * gridDim.x;
                const long long li = (long long)b2 * lines + l;
                const size_t off = a.pf && b2 < a.pf_nblk && li < a.pf_total ? (size_t)li * 128 : 0;
                pfs += *reinterpret_cast<const int*>(pb + off);
            }
        }
        // (PRO_RACE: a.pos holds the step before's position)
        const bool rec = REC && a.rec_pos && *a.rec_pos == (a.pos ? *a.pos + (PRO == PRO_RACE ? 1 : 0) : -2);
        i64 ex, ls = 0, e2 = 0, sx = 0, nn = 0;
        double sig = 1.0;
        if constexpr (PRO == PRO_ATT || PRO == PRO_PATT) att_row<NT, PRO == PRO_PATT>(a, tid, row, nbq, fz, rec);
        if constexpr (PRO == PRO_RACE) race_row<NT>(a, tid, row, nbq, ngq, bestv, besti, &race_tok);
        if constexpr (PRO == PRO_PGAUGE)
            prologue_py<NT, FG>(a, tid, row, ngq, nbq, xh_s, xl_s, red, xf_s, ex, rec && blockIdx.x == 0);
        else
            prologue<NIN, NT, PRO == PRO_RACE ? PRO_GAUGE : PRO, MODE, TOP>(a, tid, row, xh_s, xl_s, red, xf_s, ex, ls, e2,
                                                                          sx, sig, nn, rec && blockIdx.x == 0);
        const i64 fe = wsub(0, ls) & 0xFFFF;          // the fine part of (we + ex + 16) 65536 - LS for every column
        const i64 np = wsub(sx, nn);                  // EPI_TOP1: the sum of the light's positive values
        int it = 0;                                   // EPI_TOP1: tiles this wave has finished
        auto finish = [&](const v4i (&w)[U], const v4i (&w2)[U2], i64 wec, i64 bc, i64 swc, int t) {
            i64 part = wtile_partial<NIN, TC, U, WB>(w, xh_s, xl_s, lane);
            if constexpr (SPLIT) part -= wtile_partial<NIN, TC, U, WB>(w2, xh_s, xl_s, lane);   // x . W - x . W2
            i64 pile = wave_colsum64<TC>(part);
            if (INV) pile = wsub(pile, wadd(wadd(sx, swc), NIN));      // the plain pile
            const int j = t * TC + col;
            if (TOP && fin && j < a.nout) {
                // the pile lies in [C + 255 nn, C + 255 np] (the low byte w & 255 is in [0, 255]); power never
                // decreases in its argument while X EXP2 + half stays below 2^63 and the shift is a right shift,
                // so each end's score bounds the word's score (base2_stream_fr.swift:8-12); otherwise the word
                // is unsure: always a candidate, and no low
                const i64 F = wsub(wmul(wec + ex + 16, 65536), ls), sft = wsub(16, F >> 16);
                const i64 xlo = wadd(pile, wmul(255, nn)), xhi = wadd(pile, wmul(255, np));
                const bool sure = sft >= 0 && sft <= 62 && iabs64(xlo) < ((i64)1 << 44) && iabs64(xhi) < ((i64)1 << 44);
                i64 lo = INT64_MIN, hi = INT64_MAX;
                if (sure) {
                    lo = wadd(rsh(xlo * e2, sft), bc);
                    hi = wadd(rsh(xhi * e2, sft), bc);
                }
                const int k = (wave * TOP_ITERS + it) * TC + col;
                top_j[k] = j;
                top_h[k] = hi;
                top_c[k] = pile;
                best_v = max(best_v, lo);
            } else if (fin && j < a.nout) {
                if (rec && a.rpile) a.rpile[j] = pile;
                if (EPI == EPI_PILE) {
                    a.Y[j] = pile;
                } else if (EPI == EPI_PLAIN_ADD) {
                    if (a.err && pyshift_fails(pile, -(wec + ex + 16))) atomicOr(a.err, SM_ERR_RANGE);
                    const i64 add = wadd(rsh(pile, -(wec + ex + 16)), bc);
                    const i64 yb = INV ? a.Yb[j] : swc;          // (the plain machine's row was fetched with the tile)
                    const i64 r = INV ? wsub(yb, add) : wadd(yb, add);
                    a.Y[j] = r;
                    if (rec && a.rout) a.rout[j] = INV ? ~r : r;
                } else if (EPI == EPI_PLAIN || EPI == EPI_PLAIN_EDGE || EPI == EPI_PHEAD) {
                    if (a.err && pyshift_fails(pile, -(wec + ex + 16))) atomicOr(a.err, SM_ERR_RANGE);
                    i64 y = rsh(pile, -(wec + ex + 16));
                    if (EPI != EPI_PHEAD) y = wadd(y, bc);
                    if (EPI == EPI_PHEAD) {
                        if (rec && a.rlogits) a.rlogits[j] = y;
                        if (best_i < 0 || y > best_v) { best_v = y; best_i = j; }   // j grows: ties keep the first
                    } else {
                        if (rec && a.rout) a.rout[j] = y;
                        if (EPI == EPI_PLAIN_EDGE) {
                            y = FE ? edge_erf(y) : edge1(y, a.tb);
                            if (rec && a.rout2) a.rout2[j] = y;
                        }
                        a.Y[j] = y;
                    }
                } else {
                    i64 y;
                    if (FG && EPI == EPI_HEAD)          // base2.py:112-113
                        y = (i64)rint((ldexp((double)pile, (int)(wec + ex)) / sig + (double)bc * (1.0 / 65536.0)) * 65536.0);
                    else if (FG)                        // base2.py:68-69
                        y = wadd((i64)rint(ldexp((double)pile, (int)(wec + ex)) / sig * 65536.0), bc);
                    else
                        y = wadd(power_e(pile, wsub(wmul(wec + ex + 16, 65536), ls), fe, e2, a.tb), bc);
                    if (EPI == EPI_GAUGED_EDGE) y = FE ? edge_tanh(y) : edge1(y, a.tb);
                    if (EPI == EPI_HEAD) {
                        if (rec && a.rlogits) a.rlogits[j] = y;
                        const i64 u = INV ? ~y : y;                                 // the logit as the race reads it
                        if (race_beats<INV>(u, j, best_v, best_i)) { best_v = u; best_i = j; }   // j grows
                    } else {
                        a.Y[j] = y;
                        if (rec && a.rout) a.rout[j] = y;
                    }
                }
            }
        };
        if (a.ntiles <= nw) {
            // (uniform) one tile a wave, as every layer phase's grid gives: no second fetch.  The loop below would
            // request the last tile again (clamped) for the wave's empty second slot, and the launch would wait for
            // those loads at its end: 0.2422-0.2426 against 0.2498-0.2500 ms a step without them
            if (tile < a.ntiles) finish(wA, wA2, eA, bA, sA, tile);
        } else while (tile < a.ntiles) {
            const int t1 = tile + nw;
            fetch(wB, wB2, eB, bB, sB, t1);
            finish(wA, wA2, eA, bA, sA, tile);
            it++;
            if (t1 >= a.ntiles) break;
            const int t2 = t1 + nw;
            fetch(wA, wA2, eA, bA, sA, t2);
            finish(wB, wB2, eB, bB, sB, t1);
            it++;
            tile = t2;
        }
        asm volatile("" ::"v"(pfs));                    // the prefetches stay (and are done with by here)
    }
    if constexpr (TOP) {
        // the block's best low; its candidates are its words whose high reaches it (the winner's high reaches
        // the grid's best low, which is at least this one), written to the block's slots with their count
        const i64 wl = wave_reduce64(best_v, OpMax());
        if (lane == 0) bestv[wave] = wl;
        __syncthreads();
        i64 bl = bestv[0];
#pragma unroll
        for (int w = 1; w < WPB; w++) bl = max(bl, bestv[w]);
        // gathered in LDS, then written in order of falling high (rank = the candidates above it; equal highs in
        // gathering order), so that the second stage stops reading a block at its first high below the grid's
        // best low
        __shared__ int cj_s[TSLOTS];
        __shared__ i64 ch_s[TSLOTS], cc_s[TSLOTS];
        for (int k = tid; k < TSLOTS; k += NT) {
            if (top_j[k] >= 0 && top_h[k] >= bl) {
                const int n = atomicAdd(&top_n, 1);
                cj_s[n] = top_j[k];
                ch_s[n] = top_h[k];
                cc_s[n] = top_c[k];
            }
        }
        __syncthreads();
        const int n = top_n;
        for (int k = tid; k < n; k += NT) {
            const i64 h = ch_s[k];
            int r = 0;
            for (int i = 0; i < n; i++) r += ch_s[i] > h || (ch_s[i] == h && i < k);
            const size_t o = (size_t)blockIdx.x * TSLOTS + r;
            a.cand_j[o] = cj_s[k];
            a.cand_h[o] = h;
            a.cand_c[o] = cc_s[k];
        }
        if (tid == 0) {
            a.part_v[blockIdx.x] = bl;
            a.part_i[blockIdx.x] = n;
        }
        return;
    }
    if constexpr (!HEAD) return;

    // ---- this block's part of the race (base2.py:34-40, 114): largest logit, ties to the lowest word ----
    // wave: the TC finishing lanes; block: the waves; the grid's race is its own kernel (k_race1)
#pragma unroll
    for (int o = 1; o < TC; o <<= 1) {
        const i64 ov = __shfl_xor(best_v, o, 64);
        const int oi = __shfl_xor(best_i, o, 64);
        if (race_beats<INV>(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
    }
    if (lane == 16 - TC) { bestv[wave] = best_v; besti[wave] = best_i; }
    __syncthreads();
    if (tid == 0) {
        i64 bv = 0; int bi = -1;
        for (int w = 0; w < WPB; w++)
            if (race_beats<INV>(bestv[w], besti[w], bv, bi)) { bv = bestv[w]; bi = besti[w]; }
        a.part_v[blockIdx.x] = bv;
        a.part_i[blockIdx.x] = bi;
    }
}

// The batch-1 race's end, one block of 256 threads: each thread's entry (bv, bi) raced over the block (largest,
// ties to the lowest word; INV: smallest), the word fed straight back (base2_stream.swift:143-146), the position
// advanced, and the next position's entering row R0 written (GPT-2 base2.py:103: wte[word] + wpe[p]; Pythia
// foundation0/pythia_base2.py:153: rshift(embed.w[word], -(embed.e[word] + 16))), so that the next step's first
// phase reads a plain row.  At a prompt position the next word is the prompt's.  wp: the next position's wpe row
// (GPT-2), requested by the caller early.
template <int MODEL, int INV>
SMD void race1_finish(const Race1Args& a, i64 bv, int bi, int p, int plen, const i64 (&wp)[3]) {
    __shared__ i64 bvs[4];
    __shared__ int bis[4];
    __shared__ int tok_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool known = p < plen - 1;                    // a prompt position: the next word is the prompt's
    const int q = p + 1;                                // the next position
    const bool embed = q < a.npos;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const i64 ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (race_beats<INV>(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { bvs[wave] = bv; bis[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        bv = bvs[0]; bi = bis[0];
        for (int w = 1; w < 4; w++)
            if (race_beats<INV>(bvs[w], bis[w], bv, bi)) { bv = bvs[w]; bi = bis[w]; }
        int tok;
        if (known) {
            tok = a.seq[q];
        } else {
            tok = bi;
            a.seq[q] = bi;
            a.words[q - plen] = bi;
        }
        tok_s = tok;
        *a.nwords = q - plen + 1;
        *a.pos = q;
    }
    __syncthreads();
    if (!embed) return;
    const size_t tok = (size_t)tok_s;
    if (MODEL == 0) {
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const i64 e = wadd(a.wte[tok * 768 + tid + 256 * m], wp[m]);
            a.R0[tid + 256 * m] = INV ? ~e : e;
        }
    } else {
        const i64 es = -((i64)a.ee[tok] + 16);
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const size_t i = tok * 768 + tid + 256 * m;
            a.R0[tid + 256 * m] = rsh(a.ew2 ? (i64)a.ew[i] - a.ew2[i] : (i64)a.ew[i], es);   // (split: W - W2)
        }
    }
}

// Batch 1, after the head: the race over its blocks' bests (base2.py:34-40, 114), then race1_finish.  The bests are
// requested before the position is read.
// INV = 1: the complement machine's race (smallest complemented logit) and entering row ~(wte[word] + wpe[p]).
template <int MODEL, int INV = 0>
__global__ __launch_bounds__(256) void k_race1(Race1Args a) {
    static_assert(!INV || MODEL == 0, "the complement machine is GPT-2's");
    const int tid = threadIdx.x;
    constexpr int PER = 4;                              // bests a thread reads (nblk <= 1024)
    i64 pv[PER];
    int pi[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int g = tid + 256 * k;
        pv[k] = g < a.nblk ? a.part_v[g] : 0;
        pi[k] = g < a.nblk ? a.part_i[g] : -1;
    }
    const int p = *a.pos, plen = *a.plen;
    const int q = p + 1;
    i64 wp[3] = {0, 0, 0};
    if (MODEL == 0 && q < a.npos) {
#pragma unroll
        for (int m = 0; m < 3; m++) wp[m] = a.wpe[(size_t)q * 768 + tid + 256 * m];
    }
    i64 bv = 0; int bi = -1;
#pragma unroll
    for (int k = 0; k < PER; k++)
        if (race_beats<INV>(pv[k], pi[k], bv, bi)) { bv = pv[k]; bi = pi[k]; }
    race1_finish<MODEL, INV>(a, bv, bi, p, plen, wp);
}

// The collapsing top read's second stage (base2_stream_fr.swift:12-14), batch 1 (GPT-2), one block: the grid's
// best low T over the first stage's blocks; every candidate whose high reaches T survives (a word whose high is
// below T is below the word that holds T, for sure); each survivor's 768 low bytes (w & 255, word by word) finish
// its pile exactly, C + sum x (w & 255), and its score power(pile, (we + ex + 16) 65536 - LS) + b
// (base2.py:114); the race among the survivors (largest, ties to the lowest word), then race1_finish.  The
// threshold is the best low, not the 5th-best low the reference keeps for its top-5 report: the machine needs the
// winner only.
// Three rounds of memory requests: the blocks' lows and candidate counts (with the light); each block's
// candidates from the highest high down, stopping at the first below T (a block's candidates come in order of
// falling high; the first is requested in the first request); the survivors' low bytes, four lanes a survivor (192 bytes
// each), 64 survivors a pass.  Survivors
// past TOP_LIST are finished one thread each (exact, slow: a model whose bounds hold almost nothing).  The step's
// survivors are written out (count, and the first tmax: word, exact pile, score).
#define TOP_LIST 1024
__global__ __launch_bounds__(256) void k_race_top(TopArgs t) {
    const Race1Args& a = t.r;
    __shared__ __align__(16) int x_s[768];
    __shared__ int lj[TOP_LIST];
    __shared__ i64 lc[TOP_LIST];
    __shared__ i64 red_s[4];
    __shared__ int ln_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // first requests (with each block's first candidate, its highest high)
    const int g[2] = {tid, tid + 256};                  // the first stage's blocks of this thread (nblk <= 512)
    i64 bl[2], h[2] = {INT64_MIN, INT64_MIN}, cv[2] = {0, 0};
    int nc[2], jv[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 2; k++) {
        bl[k] = g[k] < a.nblk ? a.part_v[g[k]] : INT64_MIN;
        nc[k] = g[k] < a.nblk ? a.part_i[g[k]] : 0;
        if (g[k] < a.nblk) {                            // (slot 0 is read whatever the count: it is always allocated)
            const size_t o = (size_t)g[k] * t.cap;
            h[k] = t.cand_h[o];
            jv[k] = t.cand_j[o];
            cv[k] = t.cand_c[o];
        }
    }
#pragma unroll
    for (int m = 0; m < 3; m++) x_s[tid + 256 * m] = t.tx[tid + 256 * m];
    const i64 ex = t.tf[0], ls = t.tf[1], e2 = t.tf[2];
    const int p = *a.pos, plen = *a.plen;
    const int q = p + 1;
    i64 wp[3] = {0, 0, 0};
    if (q < a.npos) {
#pragma unroll
        for (int m = 0; m < 3; m++) wp[m] = a.wpe[(size_t)q * 768 + tid + 256 * m];
    }
    if (tid == 0) ln_s = 0;
    i64 T = wave_reduce64(max(bl[0], bl[1]), OpMax());
    if (lane == 0) red_s[wave] = T;
    __syncthreads();
    T = max(max(red_s[0], red_s[1]), max(red_s[2], red_s[3]));
    // second requests: both blocks' candidates in step, until each one's high falls below T
    {
        bool on[2] = {nc[0] > 0, nc[1] > 0};
        for (int c = 0; on[0] || on[1]; c++) {
            if (c > 0) {
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    if (on[k]) {
                        const size_t o = (size_t)g[k] * t.cap + c;
                        h[k] = t.cand_h[o];
                        jv[k] = t.cand_j[o];
                        cv[k] = t.cand_c[o];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 2; k++) {
                if (on[k]) {
                    if (h[k] >= T) {
                        const int n = atomicAdd(&ln_s, 1);
                        if (n < TOP_LIST) { lj[n] = jv[k]; lc[n] = cv[k]; }
                    }
                    on[k] = h[k] >= T && c + 1 < nc[k];
                }
            }
        }
    }
    __syncthreads();
    const int ns = ln_s;
    const i64 fe = wsub(0, ls) & 0xFFFF;
    auto score = [&](int j, i64 pile) {
        return wadd(power_e(pile, wsub(wmul((i64)t.we[j] + ex + 16, 65536), ls), fe, e2, t.tb), t.bias[j]);
    };
    i64 bv = 0;
    int bi = -1;
    if (ns <= TOP_LIST) {
        // third requests: four lanes a survivor, lane q of the four its bytes 192 q .. 192 q + 191
        const int gq = lane & 3, slot = lane >> 2;
        for (int s0 = 16 * wave; s0 < ns; s0 += 64) {
            const int s = s0 + slot;
            const bool live = s < ns;
            const int j = live ? lj[s] : 0;
            const v4i* lb = reinterpret_cast<const v4i*>(t.lo + (size_t)j * 768 + 192 * gq);
            v4i d[12];
#pragma unroll
            for (int k = 0; k < 12; k++) d[k] = live ? lb[k] : v4i{0, 0, 0, 0};
            const int wej = t.we[j];
            const i64 bj = t.bias[j];
            const int4* xs = reinterpret_cast<const int4*>(x_s + 192 * gq);
            int acc = 0;
#pragma unroll
            for (int k = 0; k < 12; k++) {
                const int dw[4] = {d[k].x, d[k].y, d[k].z, d[k].w};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int4 xv = xs[4 * k + w];
                    const unsigned u = (unsigned)dw[w];
                    acc += xv.x * (int)(u & 255u) + xv.y * (int)((u >> 8) & 255u) + xv.z * (int)((u >> 16) & 255u) +
                           xv.w * (int)(u >> 24);
                }
            }
            i64 sum = acc;
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            if (live && gq == 0) {
                const i64 pile = wadd(lc[s], sum);
                const i64 y = wadd(power_e(pile, wsub(wmul((i64)wej + ex + 16, 65536), ls), fe, e2, t.tb), bj);
                if (race_beats<0>(y, j, bv, bi)) { bv = y; bi = j; }
                if (s < t.tmax) { t.tw[s] = j; t.tpile[s] = pile; t.tscore[s] = y; }
            }
        }
    } else {
        // every survivor, one thread each
#pragma unroll
        for (int k = 0; k < 2; k++) {
            for (int c = 0; c < nc[k]; c++) {
                const size_t o = (size_t)g[k] * t.cap + c;
                if (t.cand_h[o] < T) break;
                const int j = t.cand_j[o];
                const unsigned char* lb = t.lo + (size_t)j * 768;
                i64 sum = 0;
                for (int i = 0; i < 768; i++) sum += (i64)x_s[i] * lb[i];
                const i64 y = score(j, wadd(t.cand_c[o], sum));
                if (race_beats<0>(y, j, bv, bi)) { bv = y; bi = j; }
            }
        }
    }
    if (tid == 0) *t.tn = ns;
    race1_finish<0, 0>(a, bv, bi, p, plen, wp);
}

// Batch 1: the entering row of the current position (the first step of a run; later steps' rows come from the race)
template <int MODEL, int INV = 0>
__global__ __launch_bounds__(256) void k_embed1(Race1Args a) {
    static_assert(!INV || MODEL == 0, "the complement machine is GPT-2's");
    const int tid = threadIdx.x;
    const int p = *a.pos;
    const size_t tok = (size_t)a.seq[p];
    if (MODEL == 0) {
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const int i = tid + 256 * m;
            const i64 e = wadd(a.wte[tok * 768 + i], a.wpe[(size_t)p * 768 + i]);
            a.R0[i] = INV ? ~e : e;
        }
    } else {
        const i64 es = -((i64)a.ee[tok] + 16);
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const size_t i = tok * 768 + tid + 256 * m;
            a.R0[tid + 256 * m] = rsh(a.ew2 ? (i64)a.ew[i] - a.ew2[i] : (i64)a.ew[i], es);   // (split: W - W2)
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// The key cache holds a key's 64 dimensions as int16, 128 bytes a position: a +32768 (the top of to16's range,
// base2.py:24-27) is held as 32767 and its bit set in the position's 64-bit mask, which the scores add back
// (q . k = q . k' + the sum of q over the masked dimensions).  The whole wave stores one row, lane = dimension.
SMD void key_store(short* krow, i64* km, int x16, int lane) {
    krow[lane] = (short)min(x16, 32767);
    const u64 m = __ballot(x16 == 32768);
    if (lane == 0) *km = (i64)m;
}
// A value row into the cache (base2.py's attention weighs the raw int64 value): its low 32 bits into V, which holds
// every value that fits 32 bits exactly.  With V64, a row with a value past 32 bits goes there whole as well, VW
// marks each row written (whole or not) and a whole row marks its (stream, head) (vbig), whose values the attention
// then reads whole.  Without V64 a value past 32 bits is an error (SM_ERR_V32).  The whole wave stores one row,
// lane = dimension; hrow: the (stream, head) of the layer's [B][12].
SMD void v_store(const AttArgs& a, size_t hrow, int p, int lane, i64 x) {
    const size_t row = hrow * a.ctx + p;
    a.V[row * 64 + lane] = (int)x;
    const bool wide = __ballot(x < (i64)INT32_MIN || x > (i64)INT32_MAX) != 0;
    if (a.V64) {
        if (wide) a.V64[row * 64 + lane] = x;
        if (lane == 0) {
            a.VW[row] = wide;
            if (wide) atomicOr(a.vbig + hrow, 1);
        }
    } else if (wide && lane == 0) {
        atomicOr(a.err, SM_ERR_V32);
    }
}
// The (stream, head)'s mark of values past 32 bits (vbig), as a vector load issued with the cached rows and waited
// for only where the attention branches on it (a scalar load there is waited for at the kernel's start); without V64
// the load's empty range reads 0 with no memory request.
SMD int vbig_load(const AttArgs& a, size_t hrow) {
    return buf_load1(buf_rsrc(a.vbig ? a.vbig + hrow : nullptr, a.vbig ? 4u : 0u), 0);
}
// Value d of cached row s of the rows from hb (the head's first row) whole: V64 where VW marks the row, else V.
SMD i64 v_whole(const AttArgs& a, size_t hb, int s, int d) {
    const size_t row = hb + s;
    return a.VW[row] ? a.V64[row * 64 + d] : (i64)a.V[row * 64 + d];
}
// q . k' by 16-bit dot products (the one-wave short path): q = 256 qh + ql with qh = q >> 8 in [-128, 128] and
// ql = q & 255, both int16, so that over 64 dimensions sum qh k' stays below 2^28 and sum ql k' below 2^30 in
// magnitude (|k'| <= 32768): two exact int32 sums, then 256 A + B in 64 bits.
typedef short s2v __attribute__((ext_vector_type(2)));
SMD int sdot2(int a, int b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2v, a), __builtin_bit_cast(s2v, b), c, false);
}
SMD int lo16(int w) { return (w << 16) >> 16; }
SMD int hi16(int w) { return w >> 16; }
// q . k' over 16 dimensions (the block path): q as four int32 quads (dimensions 0-15), k' as 16 int16 in two
// quads of pairs (dword w of quad h: dimensions 8 h + 2 w, + 1).  Each product fits 31 bits; the sum is taken
// in 64.  (The 16-bit dot products measured slower here: the pairs of q stay live through every pass.)
SMD i64 dot16(const v4i (&q)[4], const v4i (&k)[2]) {
    i64 d = 0;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int i = 8 * h + 2 * w;
            d += (i64)(q[i >> 2][i & 3] * lo16(k[h][w])) + (i64)(q[(i + 1) >> 2][(i + 1) & 3] * hi16(k[h][w]));
        }
    return d;
}
// the masked dimensions' share: the sum of q over the set bits of mb (bit j: dimension j of the 16)
SMD i64 dot16_mask(const v4i (&q)[4], unsigned mb) {
    i64 d = 0;
    if (mb) {
#pragma unroll
        for (int j = 0; j < 16; j++) d += (mb >> j) & 1 ? (i64)q[j >> 2][j & 3] : 0;
    }
    return d;
}

// ---------------------------------------------------------------------------------------------------------
// Attention for the newest position of each stream, one block per (head, stream) (base2.py:85-100).
//   1. the head's q, k through their own water level (base2.py:93); k16, ek and the raw v go to the cache
//   2. scores over every cached position s <= p: rshift(q16 . k16, -(eq + ek + 7))          (base2.py:94)
//   3. the clock starts at the maximum; arrivals ARR[max - sc] (0 past the table)            (base2.py:96-97)
//   4. num = sum a v, out = power(num, -log2fix(sum a))                                        (base2.py:98-99)
// Four lanes share a position (16 of its 64 dimensions each), so a block covers 64 positions per pass.  The
// cached keys and values of the first 64 positions are requested at launch, before the new q, k, v arrive.
// The maximum is global over the row before any arrival is read (two passes, scores in LDS), so the result is
// exact for any context length.
// The short-context path (position p < 64, one stream): one wave does a head alone, with no block barrier.
// Lane s < p holds cached key row s (prefetched at launch) and scores it against q, which every lane reads from
// LDS (the wave's own writes, read back in order); lane p is the new position (its score is a wave sum); the
// maximum and the arrival sum are wave reductions; lane d accumulates output dimension d from its prefetched V
// column, the arrivals read back from LDS the same way.  Same numbers as the general path below
// (base2.py:93-99 / pythia_base2.py:129-141).  q_s, w_s: 64 ints of LDS each.
// Returns lane's output dimension; store: this wave writes the new key and value into the cache and reports
// errors.
// The turn of one lane's value (foundation0/pythia_base2.py:116-123): dimension i < rot/2 pairs with i + rot/2;
// x' = x c - x_partner s (lower half) or x c + x_partner s (upper half).  Integer: rshift(., 30) with cos and sin
// at 2^-30; FTURN (turn=float, :118-120): round(.) in float64 with the float64 tables.
template <int FTURN>
SMD i64 turn1(i64 x, i64 partner, bool lower, i64 ci, i64 si, double cf, double sf) {
    if constexpr (FTURN) {
        const double xd = (double)x, pd = (double)partner;
        return (i64)rint(lower ? xd * cf - pd * sf : xd * cf + pd * sf);
    } else {
        return lower ? rsh(wsub(wmul(x, ci), wmul(partner, si)), 30) : rsh(wadd(wmul(x, ci), wmul(partner, si)), 30);
    }
}

template <int MODEL, int FTURN = 0, int ARRF = 0>
SMD i64 attend_short(const AttArgs& a, int p, int h, int b, int* q_s, int* w_s, i64 qv, i64 kv, const i64 vv, bool store) {
    const int lane = threadIdx.x & 63;
    const size_t hb = ((size_t)b * 12 + h) * a.ctx;         // this (stream, head)'s cache rows
    short* K16 = a.K16 + hb * 64;
    i64* KM = a.KM + hb;
    int* EK = a.EK + hb;
    int* V = a.V + hb * 64;
    // (the new q, k, v were requested by the caller before the position was read; the cached rows follow)
    // Pythia: the turn's cos and sin for dimension lane, ahead of the cached rows (lanes past rot read zeros)
    int tcos = 0, tsin = 0;
    double fcos = 0.0, fsin = 0.0;
    if constexpr (MODEL == 1) {
        const int r = a.rot >> 1, ti = lane < r ? lane : lane - r;
        if constexpr (FTURN) {
            if (lane < a.rot) { fcos = a.cosF[(size_t)p * r + ti]; fsin = a.sinF[(size_t)p * r + ti]; }
        } else {
            const unsigned lim = (unsigned)((p + 1) * r) * 4u, off = (unsigned)(p * r + ti) * 4u;
            tcos = buf_load1(buf_rsrc(a.cosT, lim), off);
            tsin = buf_load1(buf_rsrc(a.sinT, lim), off);
        }
    }
    // the cached rows s < p (lanes and columns past p read zeros without a memory request)
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(K16, (unsigned)p * 128), re = buf_rsrc(EK, (unsigned)p * 4),
                                 rm = buf_rsrc(KM, (unsigned)p * 8), rv = buf_rsrc(V, (unsigned)p * 256);
    v4i krow[8];                                             // dword w of krow[c]: dimensions 8 c + 2 w, + 1
#pragma unroll
    for (int c = 0; c < 8; c++) krow[c] = buf_load4(rk, (unsigned)lane * 128 + 16 * c);
    const int ekl = buf_load1(re, (unsigned)lane * 4);
    const u64 kml = (u64)buf_load8(rm, (unsigned)lane * 8);
    int vcol[64];
#pragma unroll
    for (int s = 0; s < 64; s++) vcol[s] = buf_load1(rv, (unsigned)(s * 64 + lane) * 4);
    const int vbg = vbig_load(a, (size_t)b * 12 + h);        // the head's values past 32 bits (read whole below)
    if constexpr (MODEL == 1) __builtin_amdgcn_sched_barrier(0);   // (the loads above stay issued here)
    if (MODEL == 1) {                                        // the turns (pythia_base2.py:116-123)
        const int r = a.rot >> 1;
        const i64 pq = __shfl(qv, lane < r ? lane + r : lane - r, 64);
        const i64 pk = __shfl(kv, lane < r ? lane + r : lane - r, 64);
        if (lane < a.rot) {
            if (!FTURN && store && (iabs64(qv) >= ((i64)1 << 31) || iabs64(kv) >= ((i64)1 << 31))) atomicOr(a.err, SM_ERR_RANGE);
            qv = turn1<FTURN>(qv, pq, lane < r, tcos, tsin, fcos, fsin);
            kv = turn1<FTURN>(kv, pk, lane < r, tcos, tsin, fcos, fsin);
        }
    }
    // the water levels of q and k (base2.py:93)
    const int shq = water_shift(wave_or64(iabs64(qv))), shk = water_shift(wave_or64(iabs64(kv)));
    const int q16 = (int)rsh(qv, shq), k16 = (int)rsh(kv, shk);
    const i64 eq = -16 + shq, ekn = -16 + shk;
    if (store) {
        key_store(K16 + (size_t)p * 64, KM + p, k16, lane);
        if (lane == 0) EK[p] = (int)ekn;
        v_store(a, (size_t)b * 12 + h, p, lane, vv);
    }
    // scores (base2.py:94): lane s < p its cached row, lane p the new key
    q_s[lane] = q16;
    // q's halves as int16 (lane = dimension) in w_s, read back as pairs (the wave's own writes, in order; the
    // arrivals overwrite w_s later): 64 16-bit dot products per lane, two exact int32 sums
    short* qh_s = reinterpret_cast<short*>(w_s);
    qh_s[lane] = (short)(q16 >> 8);
    qh_s[64 + lane] = (short)(q16 & 255);
    int A = 0, B = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const v4i qh = reinterpret_cast<const v4i*>(qh_s)[c], ql = reinterpret_cast<const v4i*>(qh_s)[8 + c];
        const v4i k = krow[c];                                         // (q: the same address in every lane)
        A = sdot2(qh.x, k.x, A); A = sdot2(qh.y, k.y, A); A = sdot2(qh.z, k.z, A); A = sdot2(qh.w, k.w, A);
        B = sdot2(ql.x, k.x, B); B = sdot2(ql.y, k.y, B); B = sdot2(ql.z, k.z, B); B = sdot2(ql.w, k.w, B);
    }
    i64 dot = 256 * (i64)A + B;
    for (u64 m = kml; m; m &= m - 1) dot += q_s[__builtin_ctzll(m)];   // the +32768 dimensions (rare)
    const i64 dn = wave_reduce64((i64)q16 * k16, OpAdd());
    const i64 ek = lane == p ? ekn : ekl;
    const i64 d = lane == p ? dn : dot;
    i64 sc = INT64_MIN;
    if (lane <= p) sc = MODEL == 1 ? rsh(wmul(d, a.ehalf), wsub(16, wsub(wmul(eq + ek + 10, 65536), a.half) >> 16))
                                   : rsh(d, -(eq + ek + 7));
    const i64 mx = wave_reduce64(sc, OpMax());
    // arrivals (base2.py:96-97) and their sum
    const int w = lane <= p ? arrival<ARRF>(a.tb, wsub(mx, sc)) : 0;
    const i64 z = wave_reduce64((i64)w, OpAdd());
    // the divisor's table entries (base2.py:99) are requested now, so their latency passes during the value sum
    int t; i64 m;
    log2_parts(z, t, m);
    const i64 F = wsub(0, wadd((i64)t * 65536, utab_log2(a.tb, (int)m)));
    const i64 hp = utab_hpow(a.tb, (int)m);
    // the value sum of dimension `lane` (base2.py:98): the cached positions s < p, then the new one
    w_s[lane] = w;
    i64 num = 0;
    int vmax = 0;
#pragma unroll
    for (int s0 = 0; s0 < 64; s0 += 8) {
        if (s0 < p) {                                        // uniform: whole groups of eight up to p
            const v4i wa = reinterpret_cast<const v4i*>(w_s)[s0 / 4], wb = reinterpret_cast<const v4i*>(w_s)[s0 / 4 + 1];
            const int wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int s = s0 + j, ws = wv[j];            // 0 for s > p
                const int vs = s < p ? vcol[s] : 0;
                num += (i64)ws * vs;
                if (MODEL == 1 && ws) vmax = max(vmax, abs(vs));
            }
        }
    }
    const int wp = __builtin_amdgcn_readlane(w, p);
    num += (i64)wp * (int)vv;
    if (MODEL == 1 && wp) vmax = max(vmax, abs((int)vv));
    double vmaxd = vmax;
    if (a.V64 && (__builtin_amdgcn_readfirstlane(vbg) || __ballot(vv < (i64)INT32_MIN || vv > (i64)INT32_MAX))) {
        // (the whole wave) the head holds a value past 32 bits: its values whole from V64, the new one from vv
        i64 n = 0, vm = 0;
        for (int s = 0; s < p; s++) {
            const int ws = w_s[s];
            const i64 x = v_whole(a, hb, s, lane);
            n = wadd(n, wmul(ws, x));
            if (MODEL == 1 && ws) vm = max(vm, iabs64(x));
        }
        num = wadd(n, wmul(wp, vv));
        if (MODEL == 1 && wp) vm = max(vm, iabs64(vv));
        vmaxd = (double)vm;
    }
    if (MODEL == 1 && store && vmaxd * (double)z >= 4611686018427387904.0) atomicOr(a.err, SM_ERR_RANGE);
    // over the total through its log (base2.py:99)
    i64 o;
    if (MODEL == 1) {
        const __int128 X = (__int128)num * hp;
        const i64 sft = 16 - (F >> 16);
        const __int128 r = sft >= 100 ? (__int128)0 : (X + ((__int128)1 << (sft - 1))) >> sft;
        if (store && (r > (__int128)INT64_MAX || r < (__int128)INT64_MIN)) atomicOr(a.err, SM_ERR_RANGE);
        o = (i64)r;
    } else {
        o = power_e(num, F, F & 0xFFFF, hp, a.tb);
    }
    return o;
}

// MODEL 1 is the Pythia machine (foundation0/pythia_base2.py:125-141): per-head interleaved q, k, v at h 192;
// the first rot dims of q and k turned by position before their water level; scores
// power(q16 . k16, (eq + ek + 10) 65536 - half); the final power exact in 128 bits (the reference's power never
// wraps, :81-85); its asserts (turn input < 2^31, max|v| sum(a) < 2^62, a result that fits) set SM_ERR_RANGE.
template <bool B> struct Flag { static constexpr bool value = B; };
#define ATT_PRE 2            // passes of 64 positions whose keys and values are requested at launch (the ring
                             // of key slots the scores loop refills two passes ahead)
// ONE = 1: one stream (the short-context path is available, full registers); ONE = 0: many streams, three waves
// a SIMD so that 768 blocks are resident at once
// REC = 0: nothing is recorded (no record position is read)
// FTURN = 1 (one stream, Pythia): turn=float
// NTB: the block's threads (256 or 512): a pass scores NTB / 4 positions (four lanes a position), the value sum
// runs NTB / 16 position groups; more threads keep more of the cache's loads in flight where the grid is small
// (h, b): the block's head and row (k_attend passes blockIdx; a paired launch its own)
// ARRF: arrivals from their formula (see arrival)
template <int MODEL, int ONE, int REC, int FTURN = 0, int NTB = NTHR, int ARRF = 0>
SMD void attend_block(const AttArgs& a, int h, int b) {
    static_assert(!FTURN || (MODEL == 1 && ONE), "turn=float is the one-stream Pythia machine's");
    static_assert(NTB == 256 || (NTB == 512 && !ONE), "256 threads, or 512 for the many-stream kernel");
    constexpr int NWB = NTB / 64, ACH = NTB / 4, NGR = NTB / 16;   // waves, positions a pass, value-sum groups
    extern __shared__ __align__(16) unsigned char smem[];
    i64* sc = reinterpret_cast<i64*>(smem);                  // [ctx] scores
    int* arr = reinterpret_cast<int*>(sc + a.ctx);           // [ctx] arrivals
    __shared__ __align__(16) int q16s[64];
    __shared__ __align__(16) int k16s[64];
    __shared__ __align__(16) int vs[64];
    __shared__ i64 vs64[64];                                // the new value whole (a head with values past 32 bits)
    __shared__ int vwide;                                   // the new value is past 32 bits
    __shared__ i64 red[8];
    __shared__ i64 numr[NGR][64];
    __shared__ int eqs, eks;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sl = tid >> 2, qd = tid & 3;                   // scores: position in the pass, lane of the position
    const int d4 = tid & 15, g = tid >> 4;                   // value sum: four dimensions, position group
    // b: the row (a stream, or a prompt position)
    // requests first (vector loads complete in order): the new q, k, v (wave w < 3 its part; in the one-stream
    // kernel wave 0 also k and v for the short path), before the position is read; then the cached keys of the
    // first ATT_PRE passes (a position's four lanes read its 128-byte row, lane qd the 32 bytes of dimensions
    // 16 qd .. + 15), their water levels and masks; the values (16 lanes a 256-byte row, four rows a wave)
    // follow once the new position is in
    const i64* qkv = a.QKV + (size_t)b * 2304;
    auto qkv_at = [&](int part) { return MODEL == 1 ? h * 192 + part * 64 + lane : part * 768 + h * 64 + lane; };
    i64 xnew = wave < 3 ? qkv[qkv_at(wave)] : 0;
    i64 xk1 = 0, xv1 = 0;
    if (ONE && wave == 0) { xk1 = qkv[qkv_at(1)]; xv1 = qkv[qkv_at(2)]; }
    const int pm = a.rowmap ? a.rowmap[b] : 0;
    const int p = a.rowmap ? pm & 0xFFFF : *a.pos, st = a.rowmap ? pm >> 16 : b;
    const bool store = !a.rowmap;                            // prompt rows: k_kv_rows stored every row's k and v
    if constexpr (ONE) {
        if (p < 64) {                                        // one stream, short context: one wave, no barriers
            if (wave == 0) {
                const i64 o = attend_short<MODEL, FTURN, ARRF>(a, p, h, b, q16s, vs, xnew, xk1, xv1, true);
                a.out[(size_t)b * 768 + h * 64 + lane] = o;
                if (a.out_or) {
                    const i64 w = wave_or64(iabs64(o));
                    if (lane == 0) a.out_or[(size_t)b * 12 + h] = w;
                }
                if (REC && b == 0 && a.rec_pos && *a.rec_pos == p) a.ratt[h * 64 + lane] = o;
            }
            return;
        }
    }
    const size_t hb = ((size_t)st * 12 + h) * a.ctx;        // this (stream, head)'s cache rows
    short* K16 = a.K16 + hb * 64;
    i64* KM = a.KM + hb;
    int* EK = a.EK + hb;
    int* V = a.V + hb * 64;
    const bool rec = REC && store && b == 0 && a.rec_pos && *a.rec_pos == p;
    const int vbg = vbig_load(a, (size_t)st * 12 + h);      // the head's values past 32 bits (read whole below)

    // Pythia: the turn's cos and sin of dimension lane (lanes < rot) with the new position, ahead of the keys, so
    // that the turn waits for them alone (row p of the [npos][rot / 2] tables; other lanes read past it: zeros)
    int tcos = 0, tsin = 0;
    double fcos = 0.0, fsin = 0.0;
    if constexpr (MODEL == 1) {
        const int r = a.rot >> 1, ti = lane < r ? lane : lane - r;
        if constexpr (FTURN) {
            if (wave < 2 && lane < a.rot) { fcos = a.cosF[(size_t)p * r + ti]; fsin = a.sinF[(size_t)p * r + ti]; }
        } else {
            const unsigned lim = (unsigned)((p + 1) * r) * 4u, off = (unsigned)(p * r + ti) * 4u;
            tcos = buf_load1(buf_rsrc(a.cosT, lim), off);
            tsin = buf_load1(buf_rsrc(a.sinT, lim), off);
        }
    }
    // (buffer loads bounded at position p: rows past it read zeros and cost no memory traffic)
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(K16, (unsigned)p * 128), re = buf_rsrc(EK, (unsigned)p * 4),
                                 rm = buf_rsrc(KM, (unsigned)p * 8), rv = buf_rsrc(V, (unsigned)p * 256);
    static_assert(ATT_PRE == 2, "the scores loop refills a ring of two key slots");
    v4i kp[ATT_PRE][2];
    int ekp[ATT_PRE];
    i64 kmp[ATT_PRE];
#pragma unroll
    for (int c = 0; c < ATT_PRE; c++) {
        const unsigned sr = sl + ACH * c;
        kp[c][0] = buf_load4(rk, sr * 128 + qd * 32);
        kp[c][1] = buf_load4(rk, sr * 128 + qd * 32 + 16);
        ekp[c] = buf_load1(re, sr * 4);
        kmp[c] = buf_load8(rm, sr * 8);
    }
    // (the loads above stay issued here, ahead of the branches that use the turn's tables)
    if constexpr (MODEL == 1) __builtin_amdgcn_sched_barrier(0);
    if (MODEL == 1 && wave < 2) {        // the turns (pythia_base2.py:116-123): pair (i, i + rot/2)
        const int r = a.rot >> 1;
        const i64 partner = __shfl(xnew, lane < r ? lane + r : lane - r, 64);
        if (lane < a.rot) {
            if (!FTURN && iabs64(xnew) >= ((i64)1 << 31)) atomicOr(a.err, SM_ERR_RANGE);
            xnew = turn1<FTURN>(xnew, partner, lane < r, tcos, tsin, fcos, fsin);
        }
    }
    // the new position's own key and value are used from LDS: this block never reads back what it wrote
    if (wave < 2) {
        const i64 x = xnew;
        const int sh = water_shift(wave_or64(iabs64(x)));
        const int x16 = (int)rsh(x, sh);
        if (wave == 0) {
            q16s[lane] = x16;
            if (lane == 0) eqs = -16 + sh;
        } else {
            k16s[lane] = x16;
            if (store) key_store(K16 + (size_t)p * 64, KM + p, x16, lane);
            if (lane == 0) {
                eks = -16 + sh;
                if (store) EK[p] = -16 + sh;
            }
        }
    } else if (wave == 2) {
        const i64 x = xnew;
        vs[lane] = (int)x;
        vs64[lane] = x;
        const bool any = __ballot(x < (i64)INT32_MIN || x > (i64)INT32_MAX) != 0;
        if (lane == 0) vwide = any;
        if (store) v_store(a, (size_t)st * 12 + h, p, lane, x);
        else if (any && !a.V64) atomicOr(a.err, SM_ERR_V32);
    }
    __syncthreads();

    // the values of positions g, g + NGR, .. of the first ATT_PRE passes, requested now: the new q and the
    // keys were ahead of them, and they arrive while the scores are formed
    constexpr int NV = ACH * ATT_PRE / NGR;
    v4i vp[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) vp[i] = buf_load4(rv, (unsigned)(g + NGR * i) * 256 + d4 * 16);

    // scores (base2.py:94 / pythia_base2.py:135) and their maximum
    const i64 eq = eqs;
    v4i qv[4];                                              // dimensions 16 qd .. + 15
#pragma unroll
    for (int u = 0; u < 4; u++) qv[u] = reinterpret_cast<const v4i*>(q16s)[4 * qd + u];
    auto score = [&](i64 dot, i64 ek) -> i64 {
        return MODEL == 1 ? rsh(wmul(dot, a.ehalf), wsub(16, wsub(wmul(eq + ek + 10, 65536), a.half) >> 16))
                          : rsh(dot, -(eq + ek + 7));
    };
    // passes of 64 positions.  Below 128 positions both passes' keys were requested at launch; beyond, two
    // passes at a time, each pass's keys requested two passes earlier into the register slot it frees (rows past
    // p read zeros and cost no memory traffic).  The two cases are separate code, so that each has exact waits.
    i64 mx = INT64_MIN;
    auto pass = [&](auto refill, int s0, v4i (&kk0)[2], int& ek0, i64& km0) {
        const int s = s0 + sl;
        i64 dot = 0, ek = ek0;
        if (s < p) {                                       // a cached key
            const v4i kk[2] = {kk0[0], kk0[1]};
            dot = dot16(qv, kk) + dot16_mask(qv, (unsigned)((u64)km0 >> (16 * qd)) & 0xFFFFu);
        } else if (s == p) {                               // the new key (int32, from LDS)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const v4i kn = reinterpret_cast<const v4i*>(k16s)[4 * qd + u];
                dot += (i64)qv[u].x * kn.x + (i64)qv[u].y * kn.y + (i64)qv[u].z * kn.z + (i64)qv[u].w * kn.w;
            }
            ek = eks;
        }
        dot += dpp64<0xB1, 0xf, 0xf>(dot, 0);              // quad_perm [1, 0, 3, 2]: the position's four lanes
        dot += dpp64<0x4E, 0xf, 0xf>(dot, 0);              // quad_perm [2, 3, 0, 1]
        if (s <= p) {
            const i64 v = score(dot, ek);
            if (qd == 0) sc[s] = v;
            mx = v > mx ? v : mx;
        }
        if constexpr (decltype(refill)::value) {          // the pass two ahead
            const unsigned sr = s0 + 2 * ACH + sl;
            kk0[0] = buf_load4(rk, sr * 128 + qd * 32);
            kk0[1] = buf_load4(rk, sr * 128 + qd * 32 + 16);
            ek0 = buf_load1(re, sr * 4);
            km0 = buf_load8(rm, sr * 8);
        }
    };
    const bool longc = p >= 2 * ACH;                       // uniform
    if (!longc) {
        pass(Flag<false>{}, 0, kp[0], ekp[0], kmp[0]);
        if (ACH <= p) pass(Flag<false>{}, ACH, kp[1], ekp[1], kmp[1]);
    } else {
        for (int s0 = 0; s0 <= p; s0 += 2 * ACH) {
            pass(Flag<true>{}, s0, kp[0], ekp[0], kmp[0]);
            if (s0 + ACH <= p) pass(Flag<true>{}, s0 + ACH, kp[1], ekp[1], kmp[1]);
        }
    }
    mx = block_reduce<OpMax, NWB>(mx, red, OpMax(), tid);   // its barriers also publish sc[]

    // arrivals (base2.py:96-97), one position per thread, into LDS; their sum
    i64 z = 0;
    for (int s = tid; s <= p; s += NTB) {
        const int w = arrival<ARRF>(a.tb, wsub(mx, sc[s]));
        arr[s] = w;
        z += w;
    }
    z = block_reduce<OpAdd, NWB>(z, red, OpAdd(), tid);     // its barriers also publish arr[]
    // the divisor's table entries (base2.py:99), requested now so that their latency passes during the value sum:
    // vector loads behind the values (scalar reads would share the LDS reads' wait counter, and the value sum's
    // first LDS read would wait for them); read unconditionally, the recomputed entries replace them where the
    // tables verified
    int zt; i64 zm;
    log2_parts(z, zt, zm);
    const int zmu = __builtin_amdgcn_readfirstlane((int)zm);
    const int zlg_mem = buf_load1(buf_rsrc(a.tb.LOG2, 65536u * 4u), (unsigned)zmu * 4u);
    const int zhp_mem = buf_load1(buf_rsrc(a.tb.HPOW, 65536u * 4u), (unsigned)zmu * 4u);

    // the value sums of dimensions 4 d4 .. + 3 over positions g, g + 16, .. (base2.py:98)
    i64 n0 = 0, n1 = 0, n2 = 0, n3 = 0;
    int vmax = 0;                               // Pythia: the largest |v| weighed (the 2^62 assert)
    auto acc = [&](int w, v4i x) {
        n0 += (i64)w * x.x; n1 += (i64)w * x.y; n2 += (i64)w * x.z; n3 += (i64)w * x.w;
        if (MODEL == 1 && w) vmax = max(vmax, max(max(abs(x.x), abs(x.y)), max(abs(x.z), abs(x.w))));
    };
    // below 2 ACH positions every value was requested after the new position came in; beyond, chunks of NGR NV
    // positions, each value requested one chunk earlier into the register slot it frees
    if (!longc) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int sv = g + NGR * i;
            if (NGR * i > p) break;                 // uniform
            if (sv < p) acc(arr[sv], vp[i]);
        }
    } else {
        for (int base = 0; base < p; base += NGR * NV) {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int sv = base + g + NGR * i;
                const v4i x = vp[i];
                vp[i] = buf_load4(rv, (unsigned)(sv + NGR * NV) * 256 + d4 * 16);
                if (sv < p) acc(arr[sv], x);
            }
        }
    }
    if (p % NGR == g) acc(arr[p], reinterpret_cast<const v4i*>(vs)[d4]);   // the new position (from LDS)
    double vmaxd = vmax;
    if (a.V64 && (__builtin_amdgcn_readfirstlane(vbg) || vwide)) {
        // (block-uniform) the head holds a value past 32 bits: its values whole, the new one from LDS
        i64 m0 = 0, m1 = 0, m2 = 0, m3 = 0, vm = 0;
        for (int sv = g; sv <= p; sv += NGR) {
            const i64 w = arr[sv];
            i64 x[4];
            for (int i = 0; i < 4; i++) x[i] = sv < p ? v_whole(a, hb, sv, 4 * d4 + i) : vs64[4 * d4 + i];
            m0 = wadd(m0, wmul(w, x[0])); m1 = wadd(m1, wmul(w, x[1])); m2 = wadd(m2, wmul(w, x[2])); m3 = wadd(m3, wmul(w, x[3]));
            if (MODEL == 1 && w) vm = max(max(vm, max(iabs64(x[0]), iabs64(x[1]))), max(iabs64(x[2]), iabs64(x[3])));
        }
        n0 = m0; n1 = m1; n2 = m2; n3 = m3;
        vmaxd = (double)vm;
    }
    if (MODEL == 1 && vmaxd * (double)z >= 4611686018427387904.0) atomicOr(a.err, SM_ERR_RANGE);
    // the NGR position groups through LDS, summed by wave 0
    numr[g][4 * d4] = n0; numr[g][4 * d4 + 1] = n1; numr[g][4 * d4 + 2] = n2; numr[g][4 * d4 + 3] = n3;
    __syncthreads();
    if (wave == 0) {
        i64 tot = 0;
#pragma unroll
        for (int i = 0; i < NGR; i++) tot += numr[i][lane];
        const i64 zlg = zlg_mem, zhp = zhp_mem;
        const i64 F = wsub(0, wadd((i64)zt * 65536, zlg));   // -log2fix(Z), the same in every lane
        i64 o;
        if (MODEL == 1) {
            // exact: (tot EXP2[f] + 2^(s-1)) >> s with s = 16 - (F >> 16) > 16 (Z >= 2^24)
            const __int128 X = (__int128)tot * zhp;
            const i64 sft = 16 - (F >> 16);
            const __int128 r = sft >= 100 ? (__int128)0 : (X + ((__int128)1 << (sft - 1))) >> sft;
            if (r > (__int128)INT64_MAX || r < (__int128)INT64_MIN) atomicOr(a.err, SM_ERR_RANGE);
            o = (i64)r;
        } else {
            o = power_e(tot, F, F & 0xFFFF, zhp, a.tb);
        }
        a.out[(size_t)b * 768 + h * 64 + lane] = o;
        if (a.out32) a.out32[(size_t)b * 768 + h * 64 + lane] = (int)o;
        if (a.out_or) {
            const i64 w = wave_or64(iabs64(o));
            if (lane == 0) a.out_or[(size_t)b * 12 + h] = w;
        }
        if (rec) a.ratt[h * 64 + lane] = o;
    }
}
template <int MODEL, int ONE, int REC, int FTURN = 0, int NTB = NTHR, int ARRF = 0>
__global__ __launch_bounds__(NTB, ONE ? 1 : 3) void k_attend(AttArgs a) {
    attend_block<MODEL, ONE, REC, FTURN, NTB, ARRF>(a, blockIdx.x, blockIdx.y);
}

// arrival=float (base2.py:89-92; foundation0/pythia_base2.py:130-133), one stream, one block per head: scores
// (q 2^-16) . (k 2^-16) / 8 in float64 against every cached key (held as float64 in KF: its raw gauged value),
// their exponentials after the row's maximum, each over their sum, out = round(sum a v).  Pythia's q and k are
// turned first (the integer turn, or FTURN).  The additions inside the dot products and sums run in this
// kernel's own order (numpy's follow its BLAS): the float arrival is compared at the word level.
// Dynamic LDS: ctx doubles.
template <int MODEL, int FTURN, int REC>
__global__ __launch_bounds__(256) void k_attend_f(AttArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    double* e_s = reinterpret_cast<double*>(smem);          // [ctx] scores, then their exponentials
    __shared__ double q_s[64], k_s[64];
    __shared__ int v_s[64];
    __shared__ double red[4];
    __shared__ double acc[4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = blockIdx.x;
    const int p = *a.pos;
    const size_t hb = (size_t)h * a.ctx;                     // stream 0's rows of head h
    double* KF = a.KF + hb * 64;
    int* V = a.V + hb * 64;
    if (wave == 0) {
        auto at = [&](int part) { return MODEL == 1 ? h * 192 + part * 64 + lane : part * 768 + h * 64 + lane; };
        i64 q = a.QKV[at(0)], k = a.QKV[at(1)];
        const i64 v = a.QKV[at(2)];
        if constexpr (MODEL == 1) {
            const int r = a.rot >> 1, ti = lane < r ? lane : lane - r;
            const i64 pq = __shfl(q, lane < r ? lane + r : lane - r, 64);
            const i64 pk = __shfl(k, lane < r ? lane + r : lane - r, 64);
            if (lane < a.rot) {
                if (!FTURN && (iabs64(q) >= ((i64)1 << 31) || iabs64(k) >= ((i64)1 << 31))) atomicOr(a.err, SM_ERR_RANGE);
                const size_t t = (size_t)p * r + ti;
                const i64 ci = FTURN ? 0 : a.cosT[t], si = FTURN ? 0 : a.sinT[t];
                const double cf = FTURN ? a.cosF[t] : 0.0, sf = FTURN ? a.sinF[t] : 0.0;
                q = turn1<FTURN>(q, pq, lane < r, ci, si, cf, sf);
                k = turn1<FTURN>(k, pk, lane < r, ci, si, cf, sf);
            }
        }
        q_s[lane] = (double)q * (1.0 / 65536.0);
        k_s[lane] = (double)k;
        v_s[lane] = (int)v;
        KF[(size_t)p * 64 + lane] = (double)k;
        if (v < (i64)INT32_MIN || v > (i64)INT32_MAX) atomicOr(a.err, SM_ERR_V32);
        V[(size_t)p * 64 + lane] = (int)v;
    }
    __syncthreads();
    // the scores (thread t: positions t, t + 256, ..; the new one from LDS) and their maximum
    double mx = -INFINITY;
    for (int j = tid; j <= p; j += 256) {
        const double* kr = j == p ? k_s : KF + (size_t)j * 64;
        double sc = 0.0;
        for (int d = 0; d < 64; d++) sc += q_s[d] * (kr[d] * (1.0 / 65536.0));
        sc = sc / 8.0;
        e_s[j] = sc;
        mx = fmax(mx, sc);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
    __syncthreads();
    // the exponentials and their sum
    double z = 0.0;
    for (int j = tid; j <= p; j += 256) {
        const double e = exp(e_s[j] - mx);
        e_s[j] = e;
        z += e;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) z += __shfl_xor(z, o, 64);
    if (lane == 0) red[wave] = z;
    __syncthreads();
    z = (red[0] + red[1]) + (red[2] + red[3]);
    // out = sum over positions of (e / z) v: wave w takes positions w, w + 4, ..; lane = dimension
    double o = 0.0;
    for (int j = wave; j <= p; j += 4) {
        const int vj = j == p ? v_s[lane] : V[(size_t)j * 64 + lane];
        o += e_s[j] / z * (double)vj;
    }
    acc[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        const i64 r = (i64)rint((acc[0][lane] + acc[1][lane]) + (acc[2][lane] + acc[3][lane]));
        a.out[h * 64 + lane] = r;
        if (REC && a.rec_pos && *a.rec_pos == p) a.ratt[h * 64 + lane] = r;
    }
}

// Prompt rows (several positions of a stream in one pass): every row's key water level and value go into the
// cache before any row's attention reads it (base2.py:93 for k; pythia_base2.py:116-123 turns k first).
// Grid (12 heads, rows), two waves: the key, the value.
template <int MODEL>
__global__ __launch_bounds__(128) void k_kv_rows(AttArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = blockIdx.x, r = blockIdx.y;
    const int pm = a.rowmap[r], st = pm >> 16, p = pm & 0xFFFF;
    const size_t at = ((size_t)st * 12 + h) * a.ctx + p;    // the row's cache slot (stream, head, position)
    i64 x = a.QKV[(size_t)r * 2304 + (MODEL == 1 ? h * 192 + (wave + 1) * 64 + lane : (wave + 1) * 768 + h * 64 + lane)];
    if (wave == 0) {
        if (MODEL == 1) {                                    // the turn, pair (i, i + rot/2)
            const int hr = a.rot >> 1;
            const i64 partner = __shfl(x, lane < hr ? lane + hr : lane - hr, 64);
            if (lane < a.rot) {
                if (iabs64(x) >= ((i64)1 << 31)) atomicOr(a.err, SM_ERR_RANGE);
                const int i = lane < hr ? lane : lane - hr;
                const i64 c = a.cosT[(size_t)p * hr + i], sn = a.sinT[(size_t)p * hr + i];
                x = lane < hr ? rsh(wsub(wmul(x, c), wmul(partner, sn)), 30) : rsh(wadd(wmul(x, c), wmul(partner, sn)), 30);
            }
        }
        const int sh = water_shift(wave_or64(iabs64(x)));
        key_store(a.K16 + at * 64, a.KM + at, (int)rsh(x, sh), lane);
        if (lane == 0) a.EK[at] = -16 + sh;
    } else {
        v_store(a, (size_t)st * 12 + h, p, lane, x);
    }
}

// ---------------------------------------------------------------------------------------------------------
// Exhaustive check of the loaded tables against their defining formulas (counts the entries that differ).
// the low 32 bits of n int64 values (a caller's rows for k_gemm's SRC path)
__global__ void k_low32(const i64* x, int* y, i64 n) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (int)x[i];
}

__global__ void k_check_tables(Tables tb, unsigned* bad) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 65536) {
        if (log2_entry(i) != tb.LOG2[i]) atomicAdd(&bad[0], 1u);
        if (exp2_entry(i) != tb.EXP2[i]) atomicAdd(&bad[1], 1u);
        if (phi_entry(i) != tb.PHI[i]) atomicAdd(&bad[2], 1u);
    }
    if (i < tb.alen && arr_entry(i) != tb.ARR[i]) atomicAdd(&bad[3], 1u);
    if (i == tb.alen && arr_entry(i) != 0) atomicAdd(&bad[3], 1u);       // the table ends where e^-d rounds to 0
}

// ---------------------------------------------------------------------------------------------------------
// Stage kernels: base2.py's stage functions on device buffers (unit parity and microbenchmarks).
__global__ void k_stage_rshift(const i64* x, const i64* s, i64* out, i64 n) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = rsh(x[i], s[i]);
}
__global__ void k_stage_power(const i64* x, const i64* F, i64* out, i64 n, Tables tb) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = power(x[i], F[i], tb);
}
__global__ void k_stage_log2fix(const i64* v, i64* out, i64 n, Tables tb) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = log2fix(v[i], tb);
}
__global__ void k_stage_edge(const i64* h, i64* out, i64 n, Tables tb) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = edge1(h[i], tb);
}
// to16 per row (one block per row); gauge != 0 also gives LS for rows of 768 (base2.py:24-27, 55-60)
__global__ __launch_bounds__(NTHR) void k_stage_rows(const i64* X, int n, int gauge, i64* x16, i64* ex, i64* LS, Tables tb) {
    __shared__ i64 red[8];
    const int tid = threadIdx.x;
    const i64* x = X + (size_t)blockIdx.x * n;
    i64 o = 0;
    for (int i = tid; i < n; i += NTHR) o |= iabs64(x[i]);
    o = block_reduce(o, red, OpOr(), tid);
    const int sh = water_shift(o);
    i64 s1 = 0, s2 = 0;
    for (int i = tid; i < n; i += NTHR) {
        const i64 v = rsh(x[i], sh);
        x16[(size_t)blockIdx.x * n + i] = v;
        s1 += v;
        s2 += v * v;
    }
    const i64 e = -16 + sh;
    if (gauge) {
        block_sum2(s1, s2, red, tid);
        if (tid == 0) LS[blockIdx.x] = gauge_ls(s1, s2, e, tb);
    }
    if (tid == 0) ex[blockIdx.x] = e;
}
// the race over n values in one block: largest, ties to the lowest index (base2.py:34-40)
__global__ __launch_bounds__(1024) void k_stage_race(const i64* v, i64 n, i64* out) {
    __shared__ i64 bvs[16];
    __shared__ i64 bis[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    i64 bv = 0, bi = -1;
    for (i64 i = tid; i < n; i += 1024) {
        const i64 x = v[i];
        if (bi < 0 || x > bv) { bv = x; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const i64 ov = __shfl_xor(bv, o, 64), oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
    }
    if (lane == 0) { bvs[wave] = bv; bis[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        bv = bvs[0]; bi = bis[0];
        for (int w = 1; w < 16; w++)
            if (bis[w] >= 0 && (bi < 0 || bvs[w] > bv || (bvs[w] == bv && bis[w] < bi))) { bv = bvs[w]; bi = bis[w]; }
        *out = bi;
    }
}

// ---------------------------------------------------------------------------------------------------------
// explicit instantiations used by the host: <NIN, TC, waves per block, prologue, epilogue, record>
#define INST(NIN, TC, WPB, PRO, EPI) template __global__ void k_gemv<NIN, TC, WPB, PRO, EPI, 0>(GemvArgs); \
    template __global__ void k_gemv<NIN, TC, WPB, PRO, EPI, 1>(GemvArgs);
INST(768, 2, 4, PRO_GAUGE, EPI_GAUGED)        // qkv
INST(768, 2, 4, PRO_RACE, EPI_GAUGED)         // layer 0's qkv with the step before's race
INST(768, 2, 2, PRO_TO16, EPI_PLAIN_ADD)      // proj
INST(768, 2, 2, PRO_ATT, EPI_PLAIN_ADD)       // proj after the attention spread over chunks (GPT-2)
INST(768, 2, 2, PRO_PATT, EPI_PLAIN_ADD)      // (Pythia)
INST(768, 2, 4, PRO_GAUGE, EPI_GAUGED_EDGE)   // fc
INST(3072, 1, 4, PRO_TO16, EPI_PLAIN_ADD)     // mproj
INST(768, 4, 4, PRO_GAUGE, EPI_HEAD)          // head (the race in its own kernel)
INST(768, 2, 4, PRO_PGAUGE, EPI_PLAIN)        // Pythia: qkv
INST(768, 2, 4, PRO_PGAUGE, EPI_PLAIN_EDGE)   // Pythia: fc
INST(768, 4, 4, PRO_PGAUGE, EPI_PHEAD)        // Pythia: head
template __global__ void k_attend<0, 0, 1>(AttArgs);
template __global__ void k_attend<0, 0, 1, 0, 512>(AttArgs);
template __global__ void k_attend<1, 0, 1, 0, 512>(AttArgs);
template __global__ void k_attend<0, 1, 0>(AttArgs);
template __global__ void k_attend<0, 1, 1>(AttArgs);
template __global__ void k_attend<1, 0, 1>(AttArgs);
template __global__ void k_attend<1, 1, 0>(AttArgs);
template __global__ void k_attend<1, 1, 1>(AttArgs);
template __global__ void k_kv_rows<0>(AttArgs);
template __global__ void k_kv_rows<1>(AttArgs);
template __global__ void k_race1<0>(Race1Args);
template __global__ void k_race1<1>(Race1Args);
template __global__ void k_embed1<0>(Race1Args);
template __global__ void k_embed1<1>(Race1Args);
// raw piles of a given light (stage entry point)
template __global__ void k_gemv<768, 2, 4, PRO_X16, EPI_PILE, 0>(GemvArgs);
template __global__ void k_gemv<768, 8, 4, PRO_X16, EPI_PILE, 0>(GemvArgs);
template __global__ void k_gemv<768, 4, 4, PRO_X16, EPI_PILE, 0>(GemvArgs);
template __global__ void k_gemv<3072, 1, 4, PRO_X16, EPI_PILE, 0>(GemvArgs);
template __global__ void k_gemv<3072, 2, 4, PRO_X16, EPI_PILE, 0>(GemvArgs);
