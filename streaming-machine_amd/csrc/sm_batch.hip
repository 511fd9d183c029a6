// Batched streams: B independent streams decoded in lockstep (one position each per step), every bank as an
// int8 MFMA contraction over byte planes (v_mfma_i32_16x16x64_i8 on gfx950).
//
// Exactness.  A light x in [-32768, 32768] is x = 256 xh + xl with xl in [0, 255]; a weight w = 256 wh + wl.
// The MFMA multiplies signed bytes, so the planes hold xh, xl' = xl - 128, wh, wl' = wl - 128 and
//   pile = 65536 HH + 256 (HL + LH) + LL + 32768 (SXh + SWh) + 128 (SXl + SWl) + 16384 K
// with HH = sum xh wh, HL = sum xh wl', LH = sum xl' wh, LL = sum xl' wl' (four MFMA accumulations, each below
// 2^26 in magnitude), SXh, SXl the light row's plane sums and SWh, SWl the plate column's.  The one light a
// byte cannot hold, xh = 128 (x = +32768), is stored as 32767 and a 0/1 correction plane c adds
// 256 sum c wh + sum c wl' + 128 sum c in the row tiles that have one.  Every pile equals base2.py's product.
//
// Operand layout (checked on the device): for a 16 x 64 A tile and a 64 x 16 B tile, lane l holds row / column
// l % 16 and bytes k = 16 (l / 16) + b, b = 0..15; the 16 x 16 result has C[4 (l / 16) + r][l % 16] in lane l.
// Plates and lights are stored in exactly that order, 1 KB per (tile, 64-k step, plane), so every operand is
// one 16-byte load per lane.
#include "sm_kernels.h"

typedef int v4i_b __attribute__((ext_vector_type(4)));

struct LightArgs {
    int K, rows;                  // row length (768 or 3072), streams
    const i64* X;                 // [rows][K] rows to light (PRO_GAUGE / PRO_TO16)
    const i64* wte; const i64* wpe; const int* seq; int seq_stride; i64* Rw;   // PRO_EMBED
    const int* pos; const int* plen;
    int skip_prompt;              // 1: nothing to do at a prompt position whose word is known (the head)
    signed char* planes;          // [RT][KS][3][64][16]: xh, xl', c
    int* rowinfo;                 // [rows][8]: ex, S1, S2 lo, S2 hi, SXh, SXl, n32768 (a gauged light's consumer
                                  // turns ex, S1, S2 into LS and the power factor, off the light's critical path)
    Tables tb;
    const int* rec_pos; i64* rx16; i64* rexls;    // stream 0's record
    // PRO_ADD_GAUGE: the producing bank's epilogue first, from its partial piles
    const i64* part; int kin;                     // [K slices][rows][K] partial piles 65536 HH + 256 MID + LL; the bank's K
    const int* csum; const int* we; const i64* bias;   // the producing plate's column facts
    i64* Y;                                       // [rows][K]: the epilogue's row (R: read and written)
    i64* rpile_in; i64* rout_in;                  // stream 0's record of the producing bank
    const int* sfacts;                            // its K slices' light facts [KSP][rows][4]: SXh, SXl, n32768, ex
    const int* rowmap;                            // prompt rows (PRO_EMBED): stream << 16 | position per row
    // PRO_RACE_EMBED: the step before's head bests [rows][nblk], the words, the counters and the position slot the
    // race writes (pos: the step before's)
    const i64* part_v; const int* part_i; int nblk;
    int* words; int words_stride; int* seqw; int* nwords; int* pos_next;
    int ls_row;                                   // gauged: slots 1-3 carry LS lo, LS hi and EXP2[-LS & 0xFFFF]
                                                  // in place of S1, S2 (the head's light)
};

struct GemmArgs {
    int K, N, rows, RT;
    const signed char* W;         // [N/16][KS][2][64][16]: wh, wl'
    const int* csum;              // [N][2]: SWh, SWl
    const int* we; const i64* bias;
    const signed char* planes; const int* rowinfo;
    i64* Y; int ystride;          // output rows [rows][ystride] (or the stream R for EPI_PLAIN_ADD)
    int* Y32;                     // EPI_GAUGED_EDGE / EPI_PLAIN_EDGE (when non-null): the outputs' low 32 bits
    Tables tb;
    const int* pos; const int* plen;
    i64* part_v; int* part_i; int nblk;   // EPI_HEAD: per (row, block) best
    const int* rec_pos; i64* rpile; i64* rout; i64* rlogits;
    i64* rout2;                   // EPI_PLAIN_EDGE: the record after the edge (rout: before it)
    i64* part;                    // EPI_PART: [ksplit][rows][N] the slice's partial pile 65536 HH + 256 MID + LL
    // the light formed in the bank (SRC > 0): the producing phase's rows, its OR words, stream 0's light record
    const i64* X; int xstride;    // [rows][xstride] int64
    const int* X32;               // the same rows' low 32 bits (read where a row's OR words show it fits 31 bits)
    const i64* orw;               // [rows][SRC]: OR of |x| over each part of a row the producer wrote
    i64* rx16; i64* rexls;
    int* sfacts;                  // EPI_PART with SRC > 0: [KSPLIT][rows][4] each K slice's SXh, SXl, n32768, ex
    i64* orw_out;                 // EPI_GAUGED_EDGE / EPI_PLAIN_EDGE (when non-null): [rows][N / 16] OR of |y| over
                                  // each block's 16 columns, the consumer's water level
    int* err;                     // the Pythia machine: its rshift assert sets SM_ERR_RANGE here
    // EPI_PLAIN_ADD2: the second plain bank, as K-slice partial piles [4][rows][N] with its K slices' light facts
    // [4][rows][4], column facts, input width; its pile and the stream after both halves for stream 0's record
    const i64* part2; const int* sfacts2; const int* csum2; const int* we2; const i64* bias2; int kin2;
    i64* rpile2; i64* rout2b;
};

// Where a bank's A operand comes from:
//   SRC = 0: the light planes and row facts a light kernel wrote (planes, rowinfo);
//   SRC = n > 0: the producing phase's int64 rows.  The producer left, per row, n OR words of the magnitudes it
//   wrote (one per attention head, say); their OR is the row's water level (base2.py:24-27), so every block
//   forms the 16-bit light of its own row tile and K steps in registers, with the plane sums its epilogue needs,
//   and no light kernel runs between the two phases.

// The light facts of a row that a K-split bank formed itself, from its slices' [KS][rows][4] (SXh, SXl, n32768
// summed; ex, the same in every slice), in the row-fact slots of a light (0: ex, 4: SXh, 5: SXl, 6: n32768)
template <int KS>
SMD void slice_facts(const int* sf, int rows, int r, int (&ri)[8]) {
    typedef int v4s __attribute__((ext_vector_type(4)));
    v4s f[KS];
#pragma unroll
    for (int q = 0; q < KS; q++) f[q] = *reinterpret_cast<const v4s*>(sf + ((size_t)q * rows + r) * 4);
    v4s t = f[0];
#pragma unroll
    for (int q = 1; q < KS; q++) t += f[q];
    ri[0] = f[0][3]; ri[1] = ri[2] = ri[3] = ri[7] = 0;
    ri[4] = t[0]; ri[5] = t[1]; ri[6] = t[2];
}

// ---------------------------------------------------------------------------------------------------------
// One block (256 threads) per stream row: the light of base2.py:24-27 (and the gauge of :55-60), written as
// MFMA A planes plus the row's exponent, gauge, power factor and plane sums.  Each thread owns groups of four
// consecutive k, so every plane byte group goes out as one 32-bit store.  KSP: the producing bank's K slices
// (PRO_ADD_GAUGE), a compile-time count so that every load of the row is in flight at once.
// The race of the step before folded into the next step's first kernel, one block a stream (k_race_rows's
// arithmetic: the largest best, ties to the lowest word).  race_load requests stream r's bests (bounded loads:
// past the last block none); race_pick reduces them over the block and returns the word fed back (a prompt
// position keeps the prompt's), block r writing it into the sequence and the words, block 0 the counters and
// the next position slot (q: the step's position, the one the word enters at).
constexpr int RACE_NB = 512;       // the head's largest grid
template <int NT>
SMD void race_load(const i64* part_v, const int* part_i, int nblk, int r, int tid, i64 (&bv)[(RACE_NB + NT - 1) / NT],
                   int (&bi)[(RACE_NB + NT - 1) / NT]) {
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(part_v + (size_t)r * nblk, (unsigned)nblk * 8u),
                                 ri = buf_rsrc(part_i + (size_t)r * nblk, (unsigned)nblk * 4u);
#pragma unroll
    for (int k = 0; k < (RACE_NB + NT - 1) / NT; k++) {
        const int g = tid + NT * k;
        bv[k] = buf_load8(rv, (unsigned)g * 8u);
        const int ci = buf_load1(ri, (unsigned)g * 4u);
        bi[k] = g < nblk ? ci : -1;
    }
}
template <int NT>
SMD int race_pick(const i64 (&rbv)[(RACE_NB + NT - 1) / NT], const int (&rbi)[(RACE_NB + NT - 1) / NT], int r, int tid,
                  int q, int plen, int* seq, int seq_stride, int* words, int words_stride, int* nwords, int* pos_next) {
    constexpr int NW = NT / 64;
    __shared__ i64 wbv[NW];
    __shared__ int wbi[NW];
    __shared__ int tok_s;
    const int lane = tid & 63, wave = tid >> 6;
    i64 bv = 0;
    int bi = -1;
#pragma unroll
    for (int k = 0; k < (RACE_NB + NT - 1) / NT; k++)
        if (rbi[k] >= 0 && (bi < 0 || rbv[k] > bv || (rbv[k] == bv && rbi[k] < bi))) { bv = rbv[k]; bi = rbi[k]; }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const i64 ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
    }
    if (lane == 0) { wbv[wave] = bv; wbi[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        bv = wbv[0]; bi = wbi[0];
        for (int w = 1; w < NW; w++)
            if (wbi[w] >= 0 && (bi < 0 || wbv[w] > bv || (wbv[w] == bv && wbi[w] < bi))) { bv = wbv[w]; bi = wbi[w]; }
        int* sq = seq + (size_t)r * seq_stride;
        const bool known = q - 1 < plen - 1;          // the step before was a prompt position
        if (!known) {
            sq[q] = bi;
            if (q - plen >= 0) words[(size_t)r * words_stride + q - plen] = bi;
        }
        if (r == 0) {
            *nwords = q - plen + 1;
            *pos_next = q;
        }
        tok_s = known ? sq[q] : bi;
    }
    __syncthreads();
    return tok_s;
}

template <int K, int PRO, int NT, int KSP>
__global__ __launch_bounds__(NT) void k_light(LightArgs a) {
    constexpr int NG = K / 4, GPT = (NG + NT - 1) / NT, KS = K / 64, NW = NT / 64;
    static_assert(NT % 64 == 0 && NW <= 12, "one to twelve waves");
    __shared__ int red[24 + 6 * 12];   // OR words [0, 24), sums [24, 96)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = blockIdx.x;
    i64 v[GPT][4];
    typedef int v4l __attribute__((ext_vector_type(4)));
    typedef i64 v2q __attribute__((ext_vector_type(2)));
    // every load of the row first: none depends on the position, so that reading it (and the prompt check)
    // overlaps them.  PRO_ADD_GAUGE: the producing bank's light facts for this row (its K slices formed the
    // light themselves), the column facts, the stream and the partial slices
    i64 i_ex = 0, i_sxh = 0, i_sxl = 0, i_n32 = 0;
    if (PRO == PRO_ADD_GAUGE) {
        int ri[8];
        slice_facts<KSP>(a.sfacts, a.rows, r, ri);
        i_ex = ri[0];
        i_sxh = ri[4]; i_sxl = ri[5]; i_n32 = ri[6];
    }
    constexpr int GA = PRO == PRO_ADD_GAUGE ? GPT : 1, KA = PRO == PRO_ADD_GAUGE ? KSP : 1;
    // PRO_RACE_EMBED: this stream's bests from the step before's head
    i64 rbv[(RACE_NB + NT - 1) / NT];
    int rbi[(RACE_NB + NT - 1) / NT];
    if constexpr (PRO == PRO_RACE_EMBED) race_load<NT>(a.part_v, a.part_i, a.nblk, r, tid, rbv, rbi);
    v4l c0[GA], c1[GA], wv[GA];
    v2q b01[GA], b23[GA], y01[GA], y23[GA], pa[GA][KA], pb[GA][KA];
#pragma unroll
    for (int m = 0; m < GPT; m++) {
        const int g = tid + NT * m;
#pragma unroll
        for (int j = 0; j < 4; j++) v[m][j] = 0;
        if (g >= NG) continue;
        const int k = 4 * g;
        if constexpr (PRO == PRO_ADD_GAUGE) {
            c0[m] = *reinterpret_cast<const v4l*>(a.csum + 2 * k); c1[m] = *reinterpret_cast<const v4l*>(a.csum + 2 * k + 4);
            wv[m] = *reinterpret_cast<const v4l*>(a.we + k);
            b01[m] = *reinterpret_cast<const v2q*>(a.bias + k); b23[m] = *reinterpret_cast<const v2q*>(a.bias + k + 2);
            y01[m] = *reinterpret_cast<const v2q*>(a.Y + (size_t)r * K + k);
            y23[m] = *reinterpret_cast<const v2q*>(a.Y + (size_t)r * K + k + 2);
#pragma unroll
            for (int ks = 0; ks < KSP; ks++) {
                const i64* q = a.part + ((size_t)ks * a.rows + r) * K + k;
                pa[m][ks] = *reinterpret_cast<const v2q*>(q);
                pb[m][ks] = *reinterpret_cast<const v2q*>(q + 2);
            }
        } else if constexpr (PRO != PRO_EMBED && PRO != PRO_RACE_EMBED) {
#pragma unroll
            for (int j = 0; j < 4; j++) v[m][j] = a.X[(size_t)r * K + k + j];
        }
    }
    // the step's position (the stage product, PRO_X16, has none; PRO_RACE_EMBED: a.pos holds the step before's)
    const int p = a.pos ? *a.pos + (PRO == PRO_RACE_EMBED ? 1 : 0) : 0;
    if (a.skip_prompt && p < *a.plen - 1) return;
    int rtok = 0;                                   // PRO_RACE_EMBED: the word fed back
    if constexpr (PRO == PRO_RACE_EMBED)
        rtok = race_pick<NT>(rbv, rbi, r, tid, p, *a.plen, a.seqw, a.seq_stride, a.words, a.words_stride, a.nwords, a.pos_next);
    const bool rec_in = r == 0 && a.rec_pos && *a.rec_pos == p;
#pragma unroll
    for (int m = 0; m < GPT; m++) {
        const int g = tid + NT * m;
        if (g >= NG) continue;
        const int k = 4 * g;
        if constexpr (PRO == PRO_ADD_GAUGE) {
            v2q s01 = pa[m][0], s23 = pb[m][0];
#pragma unroll
            for (int ks = 1; ks < KSP; ks++) { s01 += pa[m][ks]; s23 += pb[m][ks]; }
            const i64 ps[4] = {s01[0], s01[1], s23[0], s23[1]};
            const int sw[8] = {c0[m][0], c0[m][1], c0[m][2], c0[m][3], c1[m][0], c1[m][1], c1[m][2], c1[m][3]};
            const i64 bcs[4] = {b01[m][0], b01[m][1], b23[m][0], b23[m][1]}, ys[4] = {y01[m][0], y01[m][1], y23[m][0], y23[m][1]};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const i64 pile = ps[j] + 32768 * (i_sxh + sw[2 * j]) + 128 * (i_sxl + sw[2 * j + 1]) +
                                 16384 * (i64)a.kin + 128 * i_n32;
                const i64 y = wadd(ys[j], wadd(rsh(pile, -((i64)wv[m][j] + i_ex + 16)), bcs[j]));
                a.Y[(size_t)r * K + k + j] = y;
                v[m][j] = y;
                if (rec_in && a.rpile_in) a.rpile_in[k + j] = pile;
                if (rec_in && a.rout_in) a.rout_in[k + j] = y;
            }
        } else if constexpr (PRO == PRO_EMBED || PRO == PRO_RACE_EMBED) {
            const int pm = a.rowmap ? a.rowmap[r] : 0;
            const int st = a.rowmap ? pm >> 16 : r, q = a.rowmap ? pm & 0xFFFF : p;
            const i64 tok = PRO == PRO_RACE_EMBED ? rtok : a.seq[(size_t)st * a.seq_stride + q];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[m][j] = wadd(a.wte[tok * 768 + k + j], a.wpe[(i64)q * 768 + k + j]);
                a.Rw[(size_t)r * 768 + k + j] = v[m][j];
            }
        }
    }
    int sh = 0;                                     // PRO_X16: the lights are given
    if (PRO != PRO_X16) {
        u64 o = 0;
#pragma unroll
        for (int m = 0; m < GPT; m++)
#pragma unroll
            for (int j = 0; j < 4; j++) o |= (u64)iabs64(v[m][j]);
        const unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
        if (lane == 0) { red[2 * wave] = (int)olo; red[2 * wave + 1] = (int)ohi; }
        __syncthreads();
        u64 all = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) all |= ((u64)(unsigned)red[2 * w + 1] << 32) | (unsigned)red[2 * w];
        sh = water_shift((i64)all);
    }
    const i64 ex = -16 + sh;
    const bool rec = r == 0 && a.rec_pos && *a.rec_pos == p;
    int s1 = 0, sxh = 0, sxl = 0, n32 = 0;
    i64 s2 = 0;
    int* pl = reinterpret_cast<int*>(a.planes + (size_t)(r >> 4) * KS * 3 * 1024);
#pragma unroll
    for (int m = 0; m < GPT; m++) {
        const int g = tid + NT * m;
        if (g >= NG) continue;
        const int k = 4 * g;
        unsigned ph = 0, pl8 = 0, pc = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int x = (int)rsh(v[m][j], sh);
            s1 += x;
            s2 += (i64)x * x;
            if (rec && a.rx16) a.rx16[k + j] = x;
            const int c = x == 32768;
            const int xc = x - c;                  // +32768 -> 32767, the rest unchanged
            const int xh = xc >> 8, xl = (xc & 255) - 128;
            sxh += xh; sxl += xl; n32 += c;
            ph |= (unsigned)(xh & 255) << (8 * j);
            pl8 |= (unsigned)(xl & 255) << (8 * j);
            pc |= (unsigned)c << (8 * j);
        }
        const int s = k >> 6, kk = k & 63;
        const size_t off = ((size_t)s * 3 * 1024 + (size_t)((r & 15) + 16 * (kk >> 4)) * 16 + (kk & 15)) / 4;
        pl[off] = (int)ph;
        pl[off + 256] = (int)pl8;
        pl[off + 512] = (int)pc;
    }
    const int w1 = wave_add32(s1), w2h = wave_add32((int)(s2 >> 16)), w2l = wave_add32((int)(s2 & 0xFFFF));
    const int w3 = wave_add32(sxh), w4 = wave_add32(sxl), w5 = wave_add32(n32);
    if (lane == 0) { int* q = red + 24 + 6 * wave; q[0] = w1; q[1] = w2h; q[2] = w2l; q[3] = w3; q[4] = w4; q[5] = w5; }
    __syncthreads();
    if (tid == 0) {
        i64 S1 = 0, S2h = 0, S2l = 0, SXh = 0, SXl = 0, N32 = 0;
        for (int w = 0; w < NW; w++) {
            const int* q = red + 24 + 6 * w;
            S1 += q[0]; S2h += q[1]; S2l += q[2]; SXh += q[3]; SXl += q[4]; N32 += q[5];
        }
        const i64 S2 = (S2h << 16) + S2l;
        int* ri = a.rowinfo + (size_t)r * 8;
        ri[0] = (int)ex; ri[1] = (int)S1; ri[2] = (int)(u64)S2; ri[3] = (int)((u64)S2 >> 32);
        if (a.ls_row) {
            i64 e2;
            const i64 ls = gauge_ls_pow(S1, S2, ex, a.tb, e2);
            ri[1] = (int)(u64)ls; ri[2] = (int)((u64)ls >> 32); ri[3] = (int)e2;
        }
        ri[4] = (int)SXh; ri[5] = (int)SXl; ri[6] = (int)N32;
        if (rec && a.rexls) {
            i64 e2;
            a.rexls[0] = ex;
            a.rexls[1] = PRO == PRO_GAUGE || PRO == PRO_EMBED || PRO == PRO_RACE_EMBED || PRO == PRO_ADD_GAUGE
                             ? gauge_ls_pow(S1, S2, ex, a.tb, e2) : 0;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// The byte-plane contraction of a layer bank.  One block per (group of NB 16-column tiles, K slice, 16-row
// tile); its four waves split the slice's 64-k steps (NS each) and meet in LDS, where each column tile holds
// three int32 accumulators: HH, MID = HL + LH (+ CH), LL (+ CL).  Wave w then finishes rows 4 (l / 16) + w of the
// row tile for column l % 16 of every tile.  Everything the block reads that depends on nothing else (weights,
// lights, row and column facts) is issued before the first MFMA.
//   EPI_PART: the slice's partial pile 65536 HH + 256 MID + LL goes to part[kslice][rows][N]; the consumer finishes it.
//   EPI_GAUGED / EPI_GAUGED_EDGE / EPI_PLAIN_ADD / EPI_PILE: one K slice; the epilogue runs here.
// SRC > 0 (a plain epilogue or K-slice partials): each wave lights four rows of the tile from contiguous loads
// into LDS as 16-bit pairs; after one barrier every wave reads its A operands from there and forms the byte
// planes and plane sums in registers.  NB > 1 spreads that light over more columns.
// (bx, by): the block's column group / K slice and row tile (k_gemm passes blockIdx; a paired launch its own)
template <int K, int NB, int KSPLIT, int EPI, int SRC = 0>
SMD void gemm_block(const GemmArgs& a, int bx, int by) {
    constexpr int KS = K / 64, NS = KS / (4 * KSPLIT);
    constexpr bool ROWS = SRC > 0;
    static_assert(NS * 4 * KSPLIT == KS, "k steps split evenly over slices and waves");
    static_assert(KSPLIT == 1 || EPI == EPI_PART, "a split K is finished by the consumer");
    typedef int v4 __attribute__((ext_vector_type(4)));
    __shared__ int rinfo[64 * 8];
    __shared__ int red[4 * NB * 12 * 64];
    // SRC > 0: the tile's 16-bit lights as pairs [tile row][K range / 2] (rows padded by 4 dwords, so that a
    // wave's operand reads spread over the banks), each row's shift, a wave's "holds +32768" flag, and the plane
    // sums [wave][tile row] (SXh, SXl, n32768)
    constexpr int KR = K / KSPLIT, XSTR = KR / 2 + 4;
    __shared__ __align__(16) int xs[ROWS ? 16 * XSTR : 1];
    __shared__ int shs[16], cfw[4];
    __shared__ int sfx[ROWS ? 4 * 16 * 4 : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ntiles = (a.N + 15) >> 4, ngr = ntiles / NB;   // ntiles a multiple of NB
    const int nt = bx % ngr, kb = bx / ngr;                  // column group, K slice
    const int t0 = by;                                       // row tile
    const int s0 = kb * (KS / KSPLIT) + wave * NS;
    const v4* Wb = reinterpret_cast<const v4*>(a.W) + (size_t)nt * NB * KS * 128 + lane;
    const v4* Ab = reinterpret_cast<const v4*>(a.planes) + lane;
    // gauged epilogues: row tid's light facts first (loads complete in order: its gauge need not wait for the
    // tiles)
    constexpr bool GAUGED = EPI == EPI_GAUGED || EPI == EPI_GAUGED_EDGE;
    static_assert(!ROWS || !GAUGED, "a light formed here feeds a plain epilogue or K-slice partials");
    v4 gf = {0, 0, 0, 0};
    if (GAUGED) gf = *reinterpret_cast<const v4*>(a.rowinfo + (size_t)(tid < a.rows ? tid : 0) * 8);
    // SRC = 0: the row facts for LDS and each row's n32768, as bounded loads (rows past the last read zeros with
    // no traffic), so that no guarded load makes the first use wait for everything issued after it
    int n32 = 0, rsv = 0, rsv2 = 0;
    if constexpr (!ROWS) {
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(a.rowinfo, (unsigned)(a.rows * 8) * 4u);
        n32 = buf_load1(rr, (unsigned)(lane * 8 + 6) * 4u);
        rsv = buf_load1(rr, (unsigned)tid * 4u);
        rsv2 = buf_load1(rr, (unsigned)(tid + 256) * 4u);
    }
    // the column facts of each tile (for the epilogue)
    i64 swh[NB], swl[NB], we[NB], bc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) swh[nb] = swl[nb] = we[nb] = bc[nb] = 0;
    if constexpr (EPI != EPI_PART) {     // bounded loads: columns past N read zeros
        const unsigned n = (unsigned)a.N;   // csum: int32 pairs, we: int32, bias: int64
        const __amdgpu_buffer_rsrc_t rc = buf_rsrc(a.csum, 8u * n), rw = buf_rsrc(a.we, 4u * n), rb = buf_rsrc(a.bias, 8u * n);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const unsigned j = (unsigned)((nt * NB + nb) * 16 + (lane & 15));
            swh[nb] = buf_load1(rc, 8u * j); swl[nb] = buf_load1(rc, 8u * j + 4u);
            we[nb] = buf_load1(rw, 4u * j); bc[nb] = buf_load8(rb, 8u * j);
        }
    }
    v4 wh[NB][NS], wl[NB][NS], xh[NS], xl[NS];
    // SRC > 0: wave w lights tile rows 4 w .. 4 w + 3.  Their OR words (word n = lane + 64 m of the wave's
    // 4 SRC), then their values' 32-bit copies as contiguous 1 KB wave loads (values 4 (64 c + lane) .. + 3 of
    // row j), all ahead of the weights (their wait then leaves the weights in flight); rows past the last read
    // zeros.  A row whose OR words reach 2^31 is read again at 64 bits (rare: its 32-bit copy is not the value).
    constexpr int NWD = ROWS ? (4 * SRC + 63) / 64 : 1, NCH = ROWS ? KR / 128 : 1, NCH4 = ROWS ? KR / 256 : 1;
    static_assert(!ROWS || KR % 256 == 0, "a K slice of whole 256-value chunks");
    const int tr = lane & 15, q4 = lane >> 4;
    i64 ow[NWD];
    v4 xr[ROWS ? 4 : 1][NCH4];
    const int row0 = 16 * t0 + 4 * wave;
    if constexpr (ROWS) {
        const __amdgpu_buffer_rsrc_t ro = buf_rsrc(a.orw, (unsigned)(a.rows * SRC) * 8u);
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.X32, (unsigned)(a.rows * a.xstride) * 4u);
#pragma unroll
        for (int m = 0; m < NWD; m++) {
            const int n = lane + 64 * m;
            const unsigned off = n < 4 * SRC ? (unsigned)((row0 + n / SRC) * SRC + n % SRC) * 8u : 0x80000000u;
            ow[m] = (i64)__builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(ro, (int)off, 0, 0));
        }
#pragma unroll
        for (int jr = 0; jr < 4; jr++)
#pragma unroll
            for (int c = 0; c < NCH4; c++)
                xr[jr][c] = buf_load4(rx, (unsigned)((row0 + jr) * a.xstride + kb * KR + 4 * (64 * c + lane)) * 4u);
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int i = 0; i < NS; i++) {
            wh[nb][i] = __builtin_nontemporal_load(Wb + (size_t)nb * KS * 128 + (size_t)(s0 + i) * 128);
            wl[nb][i] = __builtin_nontemporal_load(Wb + (size_t)nb * KS * 128 + (size_t)(s0 + i) * 128 + 64);
        }
    // a plain bank added into the stream: the stream values this lane's epilogue adds to (its row, its column of
    // each tile) requested behind the tiles, so the epilogue does not wait on a fresh read (each is read and then
    // written by this lane alone); EPI_PLAIN_ADD2 also the second bank's partials and facts for them.  Bounded
    // loads: a row past the last (a padding row of the tile, whose lanes store nothing) reads zeros past a
    // buffer's end, or another row's values inside it, never outside the buffer
    constexpr bool ADD = EPI == EPI_PLAIN_ADD || EPI == EPI_PLAIN_ADD2;
    i64 oldv[NB];
    i64 p2[EPI == EPI_PLAIN_ADD2 ? NB : 1][4];
    int sf2[EPI == EPI_PLAIN_ADD2 ? 4 : 1][4];
    i64 swh2[NB], swl2[NB], we2[NB], bc2[NB];
    if constexpr (ADD) {
        const int orow = 16 * t0 + 4 * (lane >> 4) + wave;
        const unsigned nbytes = (unsigned)(a.rows * a.ystride) * 8u;
        const __amdgpu_buffer_rsrc_t ry = buf_rsrc(a.Y, nbytes);
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
            oldv[nb] = buf_load8(ry, (unsigned)(orow * a.ystride + (nt * NB + nb) * 16 + (lane & 15)) * 8u);
        if constexpr (EPI == EPI_PLAIN_ADD2) {
            const unsigned n = (unsigned)a.N;
            const __amdgpu_buffer_rsrc_t rp = buf_rsrc(a.part2, (unsigned)(4 * a.rows) * n * 8u);
            const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.sfacts2, (unsigned)(4 * a.rows * 4) * 4u);
            const __amdgpu_buffer_rsrc_t rc = buf_rsrc(a.csum2, 8u * n), rw = buf_rsrc(a.we2, 4u * n),
                                         rb = buf_rsrc(a.bias2, 8u * n);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const unsigned j = (unsigned)((nt * NB + nb) * 16 + (lane & 15));
#pragma unroll
                for (int q = 0; q < 4; q++)        // slice q's partial pile
                    p2[nb][q] = buf_load8(rp, (unsigned)((q * a.rows + orow) * (int)n + (int)j) * 8u);
                swh2[nb] = buf_load1(rc, 8u * j); swl2[nb] = buf_load1(rc, 8u * j + 4u);
                we2[nb] = buf_load1(rw, 4u * j); bc2[nb] = buf_load8(rb, 8u * j);
            }
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int c = 0; c < 4; c++) sf2[q][c] = buf_load1(rs, (unsigned)((q * a.rows + orow) * 4 + c) * 4u);
        }
    }
    if constexpr (!ROWS) {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            xh[i] = Ab[((size_t)t0 * KS + s0 + i) * 192];
            xl[i] = Ab[((size_t)t0 * KS + s0 + i) * 192 + 64];
        }
    }
    // keep every load above issued before any of the work below (the scheduler would sink the small ones past
    // the first MFMAs, where their latency shows)
    __builtin_amdgcn_sched_barrier(0);
    // SRC > 0: the light (base2.py:24-27) of the wave's rows into LDS, then each wave's A operands and plane
    // sums from there
    v4 xc[ROWS ? NS : 1];
    int l_n32 = 0;
    if constexpr (ROWS) {
        const int p = a.pos ? *a.pos : 0;
        const bool rec = a.rx16 && t0 == 0 && nt == 0 && a.rec_pos && *a.rec_pos == p;
        int mx = 0;
        // each row's water level from its OR words (uniform)
        i64 orr[4];
        int shv[4];
#pragma unroll
        for (int jr = 0; jr < 4; jr++) {
            i64 o = 0;
#pragma unroll
            for (int m = 0; m < NWD; m++)
                if ((lane + 64 * m) / SRC == jr) o |= ow[m];
            orr[jr] = wave_or64(o);
            shv[jr] = water_shift(orr[jr]);
            if (lane == 0) shs[4 * wave + jr] = shv[jr];
            if (rec && kb == 0 && wave == 0 && jr == 0 && lane == 0) { a.rexls[0] = shv[0] - 16; a.rexls[1] = 0; }
        }
        // light pair q (the slice's values 2 q, 2 q + 1) of row jr: +32768 held as 32767 (the correction plane
        // carries the rest)
        auto pair = [&](int jr, int q, int x0, int x1) {
            mx = max(mx, max(x0, x1));
            if (rec && wave == 0 && jr == 0) {           // stream 0's record
                a.rx16[kb * KR + 2 * q] = x0;
                a.rx16[kb * KR + 2 * q + 1] = x1;
            }
            return (int)__builtin_amdgcn_perm((unsigned)min(x1, 32767), (unsigned)min(x0, 32767), 0x05040100u);
        };
        bool wide = false;
#pragma unroll
        for (int jr = 0; jr < 4; jr++) {
            const int sh = shv[jr];
            const i64 half = sh ? (i64)1 << (sh - 1) : 0;   // rshift(v, sh), sh in [0, 49]: (v + half) >> sh
            int* xrow_s = xs + (4 * wave + jr) * XSTR;
            if ((u64)orr[jr] < ((u64)1 << 31)) {         // every |value| below 2^31: the 32-bit copies are the values
#pragma unroll
                for (int c = 0; c < NCH4; c++) {
                    const v4 w = xr[jr][c];
                    const int q = 2 * (64 * c + lane);
                    const int p0 = pair(jr, q, (int)(((i64)w[0] + half) >> sh), (int)(((i64)w[1] + half) >> sh));
                    const int p1 = pair(jr, q + 1, (int)(((i64)w[2] + half) >> sh), (int)(((i64)w[3] + half) >> sh));
                    *reinterpret_cast<int2*>(xrow_s + q) = int2{p0, p1};
                }
            } else {
                wide = true;
            }
        }
        // (rare) a row past 31 bits, read again at 64 bits (value pair 64 c + lane) after every other row, so
        // that the wait for these loads holds up nothing else
        if (wide) {
            const __amdgpu_buffer_rsrc_t r64 = buf_rsrc(a.X, (unsigned)(a.rows * a.xstride) * 8u);
#pragma unroll
            for (int jr = 0; jr < 4; jr++) {
                if ((u64)orr[jr] < ((u64)1 << 31)) continue;
                const int sh = shv[jr];
                const i64 half = sh ? (i64)1 << (sh - 1) : 0;
#pragma unroll
                for (int c = 0; c < NCH; c++) {
                    const v4 w = buf_load4(r64, (unsigned)((row0 + jr) * a.xstride + kb * KR + 2 * (64 * c + lane)) * 8u);
                    const int x0 = (int)(wadd((i64)(((u64)(unsigned)w[1] << 32) | (unsigned)w[0]), half) >> sh);
                    const int x1 = (int)(wadd((i64)(((u64)(unsigned)w[3] << 32) | (unsigned)w[2]), half) >> sh);
                    xs[(4 * wave + jr) * XSTR + 64 * c + lane] = pair(jr, 64 * c + lane, x0, x1);
                }
            }
        }
        const bool c_here = __ballot(mx == 32768) != 0;
        if (lane == 0) cfw[wave] = c_here;
        __syncthreads();
        // lane (tr, q4) of step i holds row tr, k = 64 (wave NS + i) + 16 q4 + b: 16-bit pairs d[n] = (b = 2n, 2n+1);
        // xh is each light's high byte, xl' = xl - 128 its low byte ^ 0x80; the plane sums by dot products with ones
        int sxh = 0, sxl = 0;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const v4* src = reinterpret_cast<const v4*>(xs + tr * XSTR + 32 * (wave * NS + i) + 8 * q4);
            const v4 d0 = src[0], d1 = src[1];
            const unsigned d[8] = {(unsigned)d0[0], (unsigned)d0[1], (unsigned)d0[2], (unsigned)d0[3],
                                   (unsigned)d1[0], (unsigned)d1[1], (unsigned)d1[2], (unsigned)d1[3]};
            unsigned qh[4], ql[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                qh[g] = __builtin_amdgcn_perm(d[2 * g + 1], d[2 * g], 0x07050301u);
                ql[g] = __builtin_amdgcn_perm(d[2 * g + 1], d[2 * g], 0x06040200u) ^ 0x80808080u;
                sxh = __builtin_amdgcn_sdot4((int)qh[g], 0x01010101, sxh, false);
                sxl = __builtin_amdgcn_sdot4((int)ql[g], 0x01010101, sxl, false);
            }
            xh[i] = v4{(int)qh[0], (int)qh[1], (int)qh[2], (int)qh[3]};
            xl[i] = v4{(int)ql[0], (int)ql[1], (int)ql[2], (int)ql[3]};
            xc[i] = v4{0, 0, 0, 0};
        }
        if (cfw[0] | cfw[1] | cfw[2] | cfw[3]) {       // a light of +32768 in the tile (rare): the correction
            const int sh = shs[tr];                      // plane, from the rows read again
            const i64 half = sh ? (i64)1 << (sh - 1) : 0;
            const i64* xrow = a.X + (size_t)(16 * t0 + tr) * a.xstride + kb * KR;
            const bool live = 16 * t0 + tr < a.rows;
#pragma unroll
            for (int i = 0; i < NS; i++) {
                unsigned cw[4] = {0, 0, 0, 0};
#pragma unroll
                for (int b = 0; b < 16; b++) {
                    const int c = live && (int)(wadd(xrow[64 * (wave * NS + i) + 16 * q4 + b], half) >> sh) == 32768;
                    l_n32 += c;
                    cw[b >> 2] |= (unsigned)c << (8 * (b & 3));
                }
                xc[i] = v4{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
            }
        }
        int f0 = sxh, f1 = sxl, f2 = l_n32;
        f0 += __shfl_xor(f0, 16, 64); f1 += __shfl_xor(f1, 16, 64); f2 += __shfl_xor(f2, 16, 64);
        f0 += __shfl_xor(f0, 32, 64); f1 += __shfl_xor(f1, 32, 64); f2 += __shfl_xor(f2, 32, 64);
        if (q4 == 0) {
            int* f = sfx + (wave * 16 + tr) * 4;
            f[0] = f0; f[1] = f1; f[2] = f2; f[3] = shs[tr] - 16;
        }
    }
    // gauged: thread r < rows turns row r's light facts into LS and the power factor (table reads in
    // flight during the contraction); they replace S1, S2 in the LDS copy of the row facts
    i64 g_ls = 0, g_e2 = 0;
    if (GAUGED)
        g_ls = gauge_ls_pow_v(gf[1], (i64)(((u64)(unsigned)gf[3] << 32) | (unsigned)gf[2]), gf[0], a.tb, g_e2);
    v4 acc[NB][3];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[nb][0] = acc[nb][1] = acc[nb][2] = v4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < NS; i++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            acc[nb][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[i], wh[nb][i], acc[nb][0], 0, 0, 0);
            acc[nb][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[i], wl[nb][i], acc[nb][1], 0, 0, 0);
            acc[nb][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[i], wl[nb][i], acc[nb][2], 0, 0, 0);
            acc[nb][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[i], wh[nb][i], acc[nb][1], 0, 0, 0);
        }
    // a +32768 light (held as 32767) adds its correction plane: SRC > 0, this wave's steps hold one; else
    // the row tile has one (row facts)
    bool corr;
    if constexpr (ROWS) corr = __ballot(l_n32 != 0) != 0;
    else corr = ((__ballot(n32 != 0) >> (16 * t0)) & 0xFFFFull) != 0;
    if (corr) {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            v4 cc;
            if constexpr (ROWS) cc = xc[i];
            else cc = Ab[((size_t)t0 * KS + s0 + i) * 192 + 128];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                acc[nb][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cc, wh[nb][i], acc[nb][1], 0, 0, 0);
                acc[nb][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cc, wl[nb][i], acc[nb][2], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int k3 = 0; k3 < 3; k3++)
#pragma unroll
            for (int q = 0; q < 4; q++) red[(((wave * NB + nb) * 3 + k3) * 4 + q) * 64 + lane] = acc[nb][k3][q];
    const bool keep1 = !GAUGED || (tid & 7) == 0 || (tid & 7) > 3;      // slots 1-3 carry LS, e2
    if (tid < a.rows * 8 && keep1) rinfo[tid] = rsv;
    if (tid + 256 < a.rows * 8 && keep1) rinfo[tid + 256] = rsv2;
    if (GAUGED && tid < a.rows) {
        rinfo[tid * 8 + 1] = (int)(u64)g_ls; rinfo[tid * 8 + 2] = (int)((u64)g_ls >> 32); rinfo[tid * 8 + 3] = (int)g_e2;
    }
    __syncthreads();
    if constexpr (ROWS && EPI == EPI_PART) {   // the slice's light facts, for the consumer that finishes the bank
        if (nt == 0 && tid < 16 && 16 * t0 + tid < a.rows) {
            const int* f = sfx + tid * 4;
            int* o = a.sfacts + ((size_t)kb * a.rows + 16 * t0 + tid) * 4;
            o[0] = f[0] + f[64] + f[128] + f[192];
            o[1] = f[1] + f[65] + f[129] + f[193];
            o[2] = f[2] + f[66] + f[130] + f[194];
            o[3] = f[3];
        }
    }
    const int row = 16 * t0 + 4 * (lane >> 4) + wave;
    if (row >= a.rows) return;
    const int p = a.pos ? *a.pos : 0;
    const bool rec = a.rec_pos && *a.rec_pos == p && row == 0;
    // the row's light facts
    const int* ri = rinfo + row * 8;
    i64 ex = ri[0], fsxh = ri[4], fsxl = ri[5], fn32 = ri[6];
    if constexpr (ROWS) {                            // from the four waves' steps
        const int* f = sfx + (row - 16 * t0) * 4;
        ex = f[3];
        fsxh = f[0] + f[64] + f[128] + f[192];
        fsxl = f[1] + f[65] + f[129] + f[193];
        fn32 = f[2] + f[66] + f[130] + f[194];
    }
    // every tile's result first (the edge's table reads of all NB tiles in flight together), then the stores
    i64 pile[NB], y1[NB], y2[NB];                   // y1: before the edge, y2: after it (the value written)
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        int fin[3];
#pragma unroll
        for (int k3 = 0; k3 < 3; k3++) {
            int sum = 0;
#pragma unroll
            for (int w = 0; w < 4; w++) sum += red[(((w * NB + nb) * 3 + k3) * 4 + wave) * 64 + lane];
            fin[k3] = sum;
        }
        if (EPI == EPI_PART) {
            const int j = (nt * NB + nb) * 16 + (lane & 15);
            if (j < a.N) {
                a.part[((size_t)kb * a.rows + row) * a.N + j] = 65536 * (i64)fin[0] + 256 * (i64)fin[1] + fin[2];
            }
            continue;
        }
        pile[nb] = 65536 * (i64)fin[0] + 256 * (i64)fin[1] + fin[2] + 32768 * (fsxh + swh[nb]) +
                   128 * (fsxl + swl[nb]) + 16384 * (i64)K + 128 * fn32;
        if (EPI == EPI_PILE) {
            y1[nb] = y2[nb] = pile[nb];
        } else if (ADD) {                              // the stream takes the plain bank (base2.py:73-76, 105)
            const int j = (nt * NB + nb) * 16 + (lane & 15);
            if (a.err && j < a.N && pyshift_fails(pile[nb], -(we[nb] + ex + 16))) atomicOr(a.err, SM_ERR_RANGE);
            y1[nb] = y2[nb] = wadd(oldv[nb], wadd(rsh(pile[nb], -(we[nb] + ex + 16)), bc[nb]));
            if constexpr (EPI == EPI_PLAIN_ADD2) {
                // the other half: its pile from the four K slices' accumulators and light facts (the sum the
                // row kernel would form), its plain result added too
                i64 ps2 = 0;
                int sxh = 0, sxl = 0, n32 = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    ps2 += p2[nb][q];
                    sxh += sf2[q][0]; sxl += sf2[q][1]; n32 += sf2[q][2];
                }
                const i64 ex2 = sf2[0][3];
                const i64 pile2 = ps2 + 32768 * ((i64)sxh + swh2[nb]) + 128 * ((i64)sxl + swl2[nb]) +
                                  16384 * (i64)a.kin2 + 128 * (i64)n32;
                if (a.err && j < a.N && pyshift_fails(pile2, -(we2[nb] + ex2 + 16))) atomicOr(a.err, SM_ERR_RANGE);
                y2[nb] = wadd(y1[nb], wadd(rsh(pile2, -(we2[nb] + ex2 + 16)), bc2[nb]));
                if (rec && j < a.N) {                    // stream 0's record
                    if (a.rpile2) a.rpile2[j] = pile2;
                    if (a.rout2b) a.rout2b[j] = y2[nb];
                }
            }
        } else if (EPI == EPI_PLAIN || EPI == EPI_PLAIN_EDGE) {   // the Pythia machine's banks (:112-114, 156)
            const int j = (nt * NB + nb) * 16 + (lane & 15);
            if (a.err && j < a.N && pyshift_fails(pile[nb], -(we[nb] + ex + 16))) atomicOr(a.err, SM_ERR_RANGE);
            y1[nb] = wadd(rsh(pile[nb], -(we[nb] + ex + 16)), bc[nb]);
            y2[nb] = EPI == EPI_PLAIN_EDGE ? edge1(y1[nb], a.tb) : y1[nb];
        } else {
            const i64 ls = (i64)(((u64)(unsigned)ri[2] << 32) | (unsigned)ri[1]);
            y1[nb] = wadd(power_known(pile[nb], wsub(wmul(we[nb] + ex + 16, 65536), ls), (i64)ri[3]), bc[nb]);
            y2[nb] = EPI == EPI_GAUGED_EDGE ? edge1(y1[nb], a.tb) : y1[nb];
        }
    }
    if (EPI == EPI_PART) return;
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int j = (nt * NB + nb) * 16 + (lane & 15);
        if (j < a.N) {
            a.Y[(size_t)row * a.ystride + j] = y2[nb];
            if ((EPI == EPI_GAUGED_EDGE || EPI == EPI_PLAIN_EDGE) && a.Y32) a.Y32[(size_t)row * a.ystride + j] = (int)y2[nb];
            if (rec) {                                   // stream 0's record
                if (a.rpile) a.rpile[j] = pile[nb];
                if (a.rout) a.rout[j] = EPI == EPI_PLAIN_EDGE || EPI == EPI_PLAIN_ADD2 ? y1[nb] : y2[nb];
                if (EPI == EPI_PLAIN_EDGE && a.rout2) a.rout2[j] = y2[nb];
            }
        }
        if ((EPI == EPI_GAUGED_EDGE || EPI == EPI_PLAIN_EDGE) && a.orw_out) {
            // the row's OR over this tile's 16 columns (the 16 lanes of a DPP row hold one row; N is a multiple
            // of 16, so all of them are here): prefix ORs, the total in lane 15
            i64 o = iabs64(y2[nb]);
            o |= dpp64<0x111, 0xf, 0xf>(o, 0);
            o |= dpp64<0x112, 0xf, 0xf>(o, 0);
            o |= dpp64<0x114, 0xf, 0xf>(o, 0);
            o |= dpp64<0x118, 0xf, 0xf>(o, 0);
            if ((lane & 15) == 15) a.orw_out[(size_t)row * ntiles + nt * NB + nb] = o;
        }
    }
}
template <int K, int NB, int KSPLIT, int EPI, int SRC = 0>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) { gemm_block<K, NB, KSPLIT, EPI, SRC>(a, blockIdx.x, blockIdx.y); }

// Paired launches of the Pythia machine's two independent halves of a layer (the parallel residual,
// foundation0/pythia_base2.py:155-157: the attention half and the MLP half read the stream row through their own
// gauges, so neither waits for the other).  Blocks [0, na) run the first body, the rest the second, each with the
// block coordinates its own launch would give it (gx: its grid's x extent); a block's branch is uniform, so each
// body's barriers stay block-wide, and each body keeps its own LDS.
//   k_gemm_pair: two 768-input banks (fc with its edge, qkv), both lit by the same row kernel
//   k_attend_mproj: the attention (one block a head and stream, 256 threads) and mproj's K-slice partials
template <int EA, int EB>
__global__ __launch_bounds__(256) void k_gemm_pair(GemmArgs a, GemmArgs b, int na, int gxa, int gxb) {
    const int i = blockIdx.x;
    if (i < na) {
        gemm_block<768, 1, 1, EA>(a, i % gxa, i / gxa);
    } else {
        const int j = i - na;
        gemm_block<768, 1, 1, EB>(b, j % gxb, j / gxb);
    }
}
template <int MODEL, int ARRF>
__global__ __launch_bounds__(256) void k_attend_mproj(AttArgs a, GemmArgs b, int na, int gxb) {
    const int i = blockIdx.x;
    if (i < na) {
        attend_block<MODEL, 0, 1, 0, 256, ARRF>(a, i % 12, i / 12);
    } else {
        const int j = i - na;
        gemm_block<3072, 3, 4, EPI_PART, 192>(b, j % gxb, j / gxb);
    }
}

// ---------------------------------------------------------------------------------------------------------
// The head (768 x vocab).  Wave w keeps row tile w's light planes in registers for the whole launch (12 steps x
// xh, xl: 96 VGPRs); the block streams its 16-column weight tiles (24 KB each; tile = block + k * grid) through
// two LDS buffers, two tiles ahead in registers, one barrier per tile.  A fetch past the end re-reads the last
// tile, which every block shares, so it stays in cache.  Each lane keeps, per row, the best of the columns it
// held (ties to the lowest); one 16-lane reduction per row at the end gives the block's part.
template <int RT, int EPI>
__global__ __launch_bounds__(256, 2) void k_head_rows(GemmArgs a) {     // two blocks a CU
    constexpr int K = 768, KS = K / 64, TV = KS * 128, PER = TV / 256;   // v4 per tile, per thread
    typedef int v4 __attribute__((ext_vector_type(4)));
    __shared__ v4 ws[2][TV];
    __shared__ v4 wf[2][16][2];       // the tile's column facts: SWh, SWl, we, -; bias lo, hi, -, -
    __shared__ i64 rc[64][3];         // per row: the pile's row terms, the power's row part, its factor
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int p = a.pos ? *a.pos : 0;
    // stream 0's record position (-1: none; both pointers may be null), read here with the position (a read
    // behind the tiles would wait for the tiles)
    const int rpos = a.rec_pos ? *a.rec_pos : -1;
    if ((EPI == EPI_HEAD || EPI == EPI_PHEAD) && p < *a.plen - 1) return;
    const int ntiles = (a.N + 15) >> 4, G = gridDim.x;
    // the row facts first (row tid): ex, LS, the power factor (EPI_HEAD: the producing light kernel turned S1, S2
    // into LS and EXP2[-LS & 0xFFFF]), the plane sums; then the first tile, the light planes, the second tile, so
    // that the first tile waits for nothing behind it (loads complete in order)
    // (bounded loads: rows past the last read zeros, with no branch whose join would wait for every load)
    const __amdgpu_buffer_rsrc_t rr = buf_rsrc(a.rowinfo, (unsigned)(a.rows * 8) * 4u);
    const v4 rf0 = buf_load4(rr, (unsigned)tid * 32u), rf1 = buf_load4(rr, (unsigned)tid * 32u + 16u);
    const int n32 = buf_load1(rr, (unsigned)(lane * 8 + 6) * 4u);    // rows 0-63 in every wave
    const v4* Wg = reinterpret_cast<const v4*>(a.W) + tid;
    // a tile's weights, and (threads 0-15) the facts of its column tid: rows of the slot r, refilled in place
    // (a copy of registers in flight would wait for every load: loads complete in order); threads past 15 read
    // the facts' zeros past the buffers' ends, with no branch and no memory request
    const __amdgpu_buffer_rsrc_t rcs = buf_rsrc(a.csum, (unsigned)a.N * 8u), rwe = buf_rsrc(a.we, (unsigned)a.N * 4u),
                                 rbi = buf_rsrc(EPI == EPI_HEAD ? (const void*)a.bias : (const void*)a.we,
                                                EPI == EPI_HEAD ? (unsigned)a.N * 8u : 0u);
    auto gfetch = [&](v4 (&r)[PER + 2], int tile) {
        const int tt = min(tile, ntiles - 1);
        const v4* src = Wg + (size_t)tt * TV;
#pragma unroll
        for (int i = 0; i < PER; i++) r[i] = __builtin_nontemporal_load(src + i * 256);
        const unsigned j = tid < 16 ? (unsigned)(tt * 16 + tid) : 0x10000000u;
        const u64 cs = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(rcs, (int)(j * 8u), 0, 0));
        const int we = (int)__builtin_amdgcn_raw_buffer_load_b32(rwe, (int)(j * 4u), 0, 0);
        const u64 bi = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(rbi, (int)(j * 8u), 0, 0));
        r[PER] = v4{(int)(unsigned)cs, (int)(unsigned)(cs >> 32), we, 0};
        r[PER + 1] = v4{(int)(unsigned)bi, (int)(unsigned)(bi >> 32), 0, 0};
    };
    v4 r0[PER + 2], r1[PER + 2];
    gfetch(r0, blockIdx.x);
    // this wave's row tile (waves past the last row tile only help to stage)
    const bool live = wave < RT;
    const int t = live ? wave : 0;
    const v4* Ab = reinterpret_cast<const v4*>(a.planes) + (size_t)t * KS * 192 + lane;
    v4 xh[KS], xl[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) { xh[s] = Ab[s * 192]; xl[s] = Ab[s * 192 + 64]; }
    // the loads stay issued in this order: the row facts would otherwise sink into the branch below that uses
    // them, behind the tiles, and a plane load moved behind the second tile would make the planes' wait cover it
    __builtin_amdgcn_sched_barrier(0);
    gfetch(r1, blockIdx.x + G);
    __builtin_amdgcn_sched_barrier(0);
    // row tid's constants: pile = 65536 HH + 256 MID + LL + C_row + 32768 SWh + 128 SWl; the gauged logit
    // power(pile, (we + ex + 16) 65536 - LS) + b = rshift(pile e2, 16 - we - (F_row >> 16)) + b with
    // F_row = (ex + 16) 65536 - LS (base2.py:70, 108); Pythia's plain logit rshift(pile, -(we + ex + 16))
    if (tid < a.rows) {
        rc[tid][0] = 32768 * (i64)rf1[0] + 128 * (i64)rf1[1] + 16384 * (i64)K + 128 * (i64)rf1[2];
        if (EPI == EPI_HEAD) {
            const i64 ls = (i64)(((u64)(unsigned)rf0[2] << 32) | (unsigned)rf0[1]);
            rc[tid][1] = wsub(wmul((i64)rf0[0] + 16, 65536), ls) >> 16;
            rc[tid][2] = rf0[3];
        } else {
            rc[tid][1] = (i64)rf0[0] + 16;
        }
    }
    // the light planes are in before the tile loop starts (the second tile stays in flight): inside the loop the
    // wait for them would otherwise be the loop's first use, and in every trip it would also wait for the tile
    // requested one half-trip earlier
#pragma unroll
    for (int s = 0; s < KS; s++) asm volatile("" ::"v"(xh[s]), "v"(xl[s]));
    const bool corr = live && ((__ballot(n32 != 0) >> (16 * t)) & 0xFFFFull);   // a +32768 light in the row tile
    const bool rec0 = rpos == p;
    i64 bv[4];
    int bi[4];
#pragma unroll
    for (int q = 0; q < 4; q++) { bv[q] = 0; bi[q] = -1; }
    auto compute = [&](const v4* w, const v4 (*wfs)[2], int tile) {
        if (!live) return;
        // HL and LH in accumulators of their own: two dependent chains of 12 instead of one of 24.  The row tile
        // with a +32768 light takes a loop of its own: a branch inside the k steps kept each step's LDS reads
        // behind the previous step's products (24.5 against 23.2 us at 64 streams)
        v4 hh = {0, 0, 0, 0}, hl = {0, 0, 0, 0}, lh = {0, 0, 0, 0}, ll = {0, 0, 0, 0};
        if (corr) {
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const v4 wh = w[s * 128 + lane], wl = w[s * 128 + 64 + lane];
                hh = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[s], wh, hh, 0, 0, 0);
                hl = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[s], wl, hl, 0, 0, 0);
                ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[s], wl, ll, 0, 0, 0);
                lh = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[s], wh, lh, 0, 0, 0);
                const v4 cc = Ab[s * 192 + 128];
                hl = __builtin_amdgcn_mfma_i32_16x16x64_i8(cc, wh, hl, 0, 0, 0);
                ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(cc, wl, ll, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const v4 wh = w[s * 128 + lane], wl = w[s * 128 + 64 + lane];
                hh = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[s], wh, hh, 0, 0, 0);
                hl = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh[s], wl, hl, 0, 0, 0);
                ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[s], wl, ll, 0, 0, 0);
                lh = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl[s], wh, lh, 0, 0, 0);
            }
        }
        const int j = tile * 16 + (lane & 15);
        if (j >= a.N) return;
        const v4 f0 = wfs[lane & 15][0], f1 = wfs[lane & 15][1];
        const i64 ccol = 32768 * (i64)f0[0] + 128 * (i64)f0[1], we = f0[2];
        const i64 bc = (i64)(((u64)(unsigned)f1[1] << 32) | (unsigned)f1[0]);
        if (EPI == EPI_PILE) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int row = 16 * t + 4 * (lane >> 4) + q;
                if (row >= a.rows) continue;
                const i64 pile = 65536 * (i64)hh[q] + 256 * ((i64)hl[q] + lh[q]) + ll[q] + rc[row][0] + ccol;
                if (rec0 && row == 0 && a.rpile) a.rpile[j] = pile;
                a.Y[(size_t)row * a.ystride + j] = pile;
            }
            return;
        }
        // the logit y = rsh(v, sh): v = pile (Pythia) or pile x the row's power factor, sh = -(we + F_row)
        // (Pythia) or 16 - we - F_row.  Where every lane's shift is in 1..62 (the usual case) rsh is the rounding
        // add and one arithmetic shift; otherwise the wave takes the general rsh (and Pythia's range check,
        // which only a left shift can fail).  Rows past the last are computed from unwritten facts and left out.
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = 16 * t + 4 * (lane >> 4) + q;
            const i64 pile = 65536 * (i64)hh[q] + 256 * ((i64)hl[q] + lh[q]) + ll[q] + rc[row][0] + ccol;
            const i64 v = EPI == EPI_PHEAD ? pile : wmul(pile, rc[row][2]);
            const i64 s = EPI == EPI_PHEAD ? -(we + rc[row][1]) : 16 - we - rc[row][1];
            i64 y;
            if (__ballot(row < a.rows && (u64)(s - 1) >= 62) == 0) {
                const int s32 = (int)s;
                y = wadd(v, (i64)1 << (s32 - 1)) >> s32;
            } else {
                if (EPI == EPI_PHEAD && row < a.rows && a.err && pyshift_fails(v, s)) atomicOr(a.err, SM_ERR_RANGE);
                y = rsh(v, s);
            }
            if (EPI == EPI_HEAD) y = wadd(y, bc);                            // Pythia's head has no bias
            if (row < a.rows && (bi[q] < 0 || y > bv[q])) { bv[q] = y; bi[q] = j; }    // j grows with the tile
            if (q == 0 && rec0 && t == 0 && lane < 16) {                   // row 0: q = 0 of lanes 0-15
                if (a.rpile) a.rpile[j] = pile;
                if (a.rlogits) a.rlogits[j] = y;
            }
        }
    };
    // (each slot is refilled in place once it is used; no exit inside the loop, so the waits stay exact)
    for (int tile = blockIdx.x; tile < ntiles;) {
#pragma unroll
        for (int i = 0; i < PER; i++) ws[0][tid + i * 256] = r0[i];
        if (tid < 16) { wf[0][tid][0] = r0[PER]; wf[0][tid][1] = r0[PER + 1]; }
        gfetch(r0, tile + 2 * G);
        __syncthreads();
        compute(ws[0], wf[0], tile);
        tile += G;                                   // (a tile past the end computes nothing)
#pragma unroll
        for (int i = 0; i < PER; i++) ws[1][tid + i * 256] = r1[i];
        if (tid < 16) { wf[1][tid][0] = r1[PER]; wf[1][tid][1] = r1[PER + 1]; }
        gfetch(r1, tile + 2 * G);
        __syncthreads();
        compute(ws[1], wf[1], tile);
        tile += G;
    }
    if ((EPI != EPI_HEAD && EPI != EPI_PHEAD) || !live) return;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        i64 v = bv[q];
        int i = bi[q];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const i64 ov = __shfl_xor(v, o, 64);
            const int oi = __shfl_xor(i, o, 64);
            if (oi >= 0 && (i < 0 || ov > v || (ov == v && oi < i))) { v = ov; i = oi; }
        }
        const int row = 16 * t + 4 * (lane >> 4) + q;
        if ((lane & 15) == 0 && row < a.rows) {
            a.part_v[(size_t)row * a.nblk + blockIdx.x] = v;
            a.part_i[(size_t)row * a.nblk + blockIdx.x] = i;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// The Pythia machine, batched (foundation0/pythia_base2.py:100-160 for every stream).  One block per stream row.
//
// four lights k .. k + 3 of row r (x = rshift(v, sh)) into the MFMA A planes of a K-wide row (xh, xl', c, each
// group of four as one 32-bit store), adding to the row's plane sums
template <int K>
SMD void planes4(const i64 (&v)[4], int sh, int r, int k, signed char* planes, bool rec, i64* rx16, int& sxh,
                 int& sxl, int& n32) {
    constexpr int KS = K / 64;
    int* pl = reinterpret_cast<int*>(planes + (size_t)(r >> 4) * KS * 3 * 1024);
    unsigned ph = 0, pq = 0, pc = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int x = (int)rsh(v[j], sh);
        if (rec && rx16) rx16[k + j] = x;
        const int c = x == 32768;
        const int xc = x - c;
        const int xh = xc >> 8, xl = (xc & 255) - 128;
        sxh += xh; sxl += xl; n32 += c;
        ph |= (unsigned)(xh & 255) << (8 * j);
        pq |= (unsigned)(xl & 255) << (8 * j);
        pc |= (unsigned)c << (8 * j);
    }
    const int s = k >> 6, kk = k & 63;
    const size_t off = ((size_t)s * 3 * 1024 + (size_t)((r & 15) + 16 * (kk >> 4)) * 16 + (kk & 15)) / 4;
    pl[off] = (int)ph;
    pl[off + 256] = (int)pq;
    pl[off + 512] = (int)pc;
}

struct PyRowArgs {
    int rows;
    i64* R;                                       // [rows][768] the stream
    const short* ew; const int* ee; const int* seq; int seq_stride; const int* pos;   // the word enters
    const int* ng1; const i64* nb1; int nge1;     // gauge 1 (ln1, or lnf at the top)
    const int* ng2; const i64* nb2; int nge2;     // gauge 2 (ln2); null: one gauge only
    signed char* planes1; int* rowinfo1;          // light of gauge 1
    signed char* planes2; int* rowinfo2;          // light of gauge 2
    // PY_ADD: mproj's four K slices of partial piles, finished here (proj's half is already in R)
    const i64* partM; int kinM; const int* csumM; const int* weM; const i64* biasM;
    const int* sfactsM;                           // mproj's K slices' light facts [4][rows][4]
    Tables tb;
    const int* rec_pos;
    i64* rg1; i64* rx1; i64* rex1; i64* rg2; i64* rx2; i64* rex2;   // the gauges and their lights
    i64* rpileM; i64* routM;                                         // PY_ADD: mproj's pile, the stream after it
    const int* rowmap;                            // prompt rows (PY_EMBED): stream << 16 | position per row
    int* err;                                     // its rshift assert (PY_ADD) sets SM_ERR_RANGE here
    // PY_RACE_EMBED: the step before's head bests [rows][nblk], the prompt length, the words, the counters and the
    // position slot the race writes (pos: the step before's)
    const i64* part_v; const int* part_i; int nblk; const int* plen;
    int* words; int words_stride; int* seqw; int* nwords; int* pos_next;
};
// PY_RACE_EMBED: the race of the step before (race_pick), then PY_EMBED of the word it feeds back
enum { PY_EMBED = 0, PY_ADD = 1, PY_GAUGE = 2, PY_RACE_EMBED = 3 };

// plain(pile) of one bank for columns k .. k + 3 of row r, from its KS K-sliced partial piles
// (:112-114), in two halves so that a caller can have every load of its row in flight before the arithmetic
typedef int v4l_p __attribute__((ext_vector_type(4)));
typedef i64 v2q_p __attribute__((ext_vector_type(2)));
template <int KS>
struct Plain4 { v2q_p pa[KS], pb[KS]; v4l_p c0, c1, wv; v2q_p b01, b23; };
template <int KS>
SMD void plain4_load(Plain4<KS>& P, const i64* part, int rows, int N, const int* csum, const int* we, const i64* bias,
                     int r, int k) {
    P.c0 = *reinterpret_cast<const v4l_p*>(csum + 2 * k);
    P.c1 = *reinterpret_cast<const v4l_p*>(csum + 2 * k + 4);
    P.wv = *reinterpret_cast<const v4l_p*>(we + k);
    P.b01 = *reinterpret_cast<const v2q_p*>(bias + k);
    P.b23 = *reinterpret_cast<const v2q_p*>(bias + k + 2);
#pragma unroll
    for (int q = 0; q < KS; q++) {
        const i64* src = part + ((size_t)q * rows + r) * N + k;
        P.pa[q] = *reinterpret_cast<const v2q_p*>(src);
        P.pb[q] = *reinterpret_cast<const v2q_p*>(src + 2);
    }
}
template <int KS>
SMD void plain4_finish(const Plain4<KS>& P, int kin, const int* ri, i64 (&pile)[4], i64 (&y)[4], int* err) {
    v2q_p s01 = P.pa[0], s23 = P.pb[0];
#pragma unroll
    for (int q = 1; q < KS; q++) { s01 += P.pa[q]; s23 += P.pb[q]; }
    const i64 ps[4] = {s01[0], s01[1], s23[0], s23[1]};
    const int sw[8] = {P.c0[0], P.c0[1], P.c0[2], P.c0[3], P.c1[0], P.c1[1], P.c1[2], P.c1[3]};
    const i64 bc[4] = {P.b01[0], P.b01[1], P.b23[0], P.b23[1]};
    const i64 ex = ri[0], sxh = ri[4], sxl = ri[5], n32 = ri[6];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        pile[j] = ps[j] + 32768 * (sxh + sw[2 * j]) + 128 * (sxl + sw[2 * j + 1]) + 16384 * (i64)kin + 128 * n32;
        if (err && pyshift_fails(pile[j], -((i64)P.wv[j] + ex + 16))) atomicOr(err, SM_ERR_RANGE);
        y[j] = wadd(rsh(pile[j], -((i64)P.wv[j] + ex + 16)), bc[j]);
    }
}

// One block per stream row.
//   PY_EMBED: R = rshift(embed.w[word], -(embed.e[word] + 16)) (:153), then the two gauges' lights
//   PY_ADD:   R += plain(mproj) (:155-157; proj's half was added by its bank), then the two gauges' lights (or
//             lnf's alone)
//   PY_GAUGE: R complete (proj's bank added both halves, EPI_PLAIN_ADD2), the two gauges' lights (or lnf's)
// Both gauges share to16(R), S1, S2 and LS (:100-110); only the gain, its power and the offset differ.  The two
// lights go through their water levels and plane sums together: four barriers in all (the OR of R, S1 and S2,
// the lights' ORs, their plane sums), each with LDS slots of its own, and the gains and offsets are requested
// with the row.
template <int MODE>
__global__ __launch_bounds__(192) void k_py_rows(PyRowArgs a) {
    constexpr int NT = 192, NW = NT / 64;
    __shared__ int red[NW * (2 + 3 + 4 + 6)];      // OR(R) | S1, S2 | OR of the two lights | their plane sums
    int* const rOR = red;
    int* const rS = red + 2 * NW;
    int* const rLO = red + 5 * NW;
    int* const rLS = red + 9 * NW;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = blockIdx.x;
    i64 rbv[(RACE_NB + NT - 1) / NT];
    int rbi[(RACE_NB + NT - 1) / NT];
    if constexpr (MODE == PY_RACE_EMBED) race_load<NT>(a.part_v, a.part_i, a.nblk, r, tid, rbv, rbi);
    const int pm = a.rowmap ? a.rowmap[r] : 0;
    // the step's position (PY_RACE_EMBED: a.pos holds the step before's)
    const int p = a.rowmap ? pm & 0xFFFF : *a.pos + (MODE == PY_RACE_EMBED ? 1 : 0), st = a.rowmap ? pm >> 16 : r;
    const bool rec = r == 0 && a.rec_pos && *a.rec_pos == p;
    const bool two = a.ng2 != nullptr;             // uniform
    // the stream row (192 threads hold four lanes each)
    const int k = 4 * tid;
    i64 R4[4] = {0, 0, 0, 0};
    int gn[2][4];
    i64 gb[2][4];
    {
        if (MODE == PY_EMBED || MODE == PY_RACE_EMBED) {
            const i64 tok = MODE == PY_RACE_EMBED
                ? race_pick<NT>(rbv, rbi, r, tid, p, *a.plen, a.seqw, a.seq_stride, a.words, a.words_stride, a.nwords, a.pos_next)
                : a.seq[(size_t)st * a.seq_stride + p];
            const i64 es = -((i64)a.ee[tok] + 16);
#pragma unroll
            for (int j = 0; j < 4; j++) R4[j] = rsh((i64)a.ew[tok * 768 + k + j], es);
        } else {
            i64 pM[4], yM[4];
            // mproj's partials (four K slices) and the stream row, all requested before any use
            Plain4<4> PM;
            if (MODE == PY_ADD) plain4_load<4>(PM, a.partM, a.rows, 768, a.csumM, a.weM, a.biasM, r, k);
            const v2q_p r01 = *reinterpret_cast<const v2q_p*>(a.R + (size_t)r * 768 + k);
            const v2q_p r23 = *reinterpret_cast<const v2q_p*>(a.R + (size_t)r * 768 + k + 2);
            const i64 rr[4] = {r01[0], r01[1], r23[0], r23[1]};
            int rim[8];
            if (MODE == PY_ADD) slice_facts<4>(a.sfactsM, a.rows, r, rim);
            // the gains and offsets (they depend on nothing here)
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                const int* ng = gi ? (two ? a.ng2 : a.ng1) : a.ng1;
                const i64* nb = gi ? (two ? a.nb2 : a.nb1) : a.nb1;
                const v4l_p g4 = *reinterpret_cast<const v4l_p*>(ng + k);
                const v2q_p b01 = *reinterpret_cast<const v2q_p*>(nb + k), b23 = *reinterpret_cast<const v2q_p*>(nb + k + 2);
                gn[gi][0] = g4[0]; gn[gi][1] = g4[1]; gn[gi][2] = g4[2]; gn[gi][3] = g4[3];
                gb[gi][0] = b01[0]; gb[gi][1] = b01[1]; gb[gi][2] = b23[0]; gb[gi][3] = b23[1];
            }
            if (MODE == PY_ADD) {
                plain4_finish<4>(PM, a.kinM, rim, pM, yM, a.err);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    R4[j] = wadd(rr[j], yM[j]);
                    if (rec) {
                        if (a.rpileM) a.rpileM[k + j] = pM[j];
                        if (a.routM) a.routM[k + j] = R4[j];
                    }
                }
            } else {                                     // PY_GAUGE: the stream is complete
#pragma unroll
                for (int j = 0; j < 4; j++) R4[j] = rr[j];
            }
        }
        if (MODE == PY_EMBED || MODE == PY_RACE_EMBED) {
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                const int* ng = gi ? (two ? a.ng2 : a.ng1) : a.ng1;
                const i64* nb = gi ? (two ? a.nb2 : a.nb1) : a.nb1;
#pragma unroll
                for (int j = 0; j < 4; j++) { gn[gi][j] = ng[k + j]; gb[gi][j] = nb[k + j]; }
            }
        }
        if (MODE != PY_GAUGE) {
#pragma unroll
            for (int j = 0; j < 4; j++) a.R[(size_t)r * 768 + k + j] = R4[j];
        }
    }
    // the gauge (:100-110): to16(R), S1, S2, LS, the power factor
    u64 o = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) o |= (u64)iabs64(R4[j]);
    unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
    if (lane == 0) { rOR[2 * wave] = (int)olo; rOR[2 * wave + 1] = (int)ohi; }
    __syncthreads();
    u64 all = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) all |= ((u64)(unsigned)rOR[2 * w + 1] << 32) | (unsigned)rOR[2 * w];
    const int sh = water_shift((i64)all);
    int x[4];
    int s1 = 0;
    i64 s2 = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        x[j] = (int)rsh(R4[j], sh);
        s1 += x[j];
        s2 += (i64)x[j] * x[j];
    }
    const int w1 = wave_add32(s1), w2h = wave_add32((int)(s2 >> 16)), w2l = wave_add32((int)(s2 & 0xFFFF));
    if (lane == 0) { rS[3 * wave] = w1; rS[3 * wave + 1] = w2h; rS[3 * wave + 2] = w2l; }
    __syncthreads();
    i64 S1 = 0, S2h = 0, S2l = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) { S1 += rS[3 * w]; S2h += rS[3 * w + 1]; S2l += rS[3 * w + 2]; }
    i64 e2;
    const i64 ls = pgauge_ls_pow(S1, (S2h << 16) + S2l, -16 + sh, a.tb, e2);
    // the two gauged rows (:109-110): rshift((768 x - S1) g e2, sg) + offset
    i64 v[2][4];
    u64 og[2] = {0, 0};
#pragma unroll
    for (int gi = 0; gi < 2; gi++) {
        const i64 sg = wsub(16, wsub(wmul((i64)(gi && two ? a.nge2 : a.nge1) + 16, 65536), ls) >> 16);
        i64* rg = gi ? a.rg2 : a.rg1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const i64 c = 768 * (i64)x[j] - S1;
            v[gi][j] = wadd(rsh(wmul(c * gn[gi][j], e2), sg), gb[gi][j]);
            if (rec && rg && (gi == 0 || two)) rg[k + j] = v[gi][j];
            og[gi] |= (u64)iabs64(v[gi][j]);
        }
    }
    // their water levels
#pragma unroll
    for (int gi = 0; gi < 2; gi++) {
        const unsigned lo = wave_or32((unsigned)og[gi]), hi = wave_or32((unsigned)(og[gi] >> 32));
        if (lane == 0) { rLO[4 * wave + 2 * gi] = (int)lo; rLO[4 * wave + 2 * gi + 1] = (int)hi; }
    }
    __syncthreads();
    int shg[2], fs[2][3];
#pragma unroll
    for (int gi = 0; gi < 2; gi++) {
        u64 ag = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) ag |= ((u64)(unsigned)rLO[4 * w + 2 * gi + 1] << 32) | (unsigned)rLO[4 * w + 2 * gi];
        shg[gi] = water_shift((i64)ag);
        fs[gi][0] = fs[gi][1] = fs[gi][2] = 0;
        if (gi == 0 || two)
            planes4<768>(v[gi], shg[gi], r, k, gi ? a.planes2 : a.planes1, rec, gi ? a.rx2 : a.rx1, fs[gi][0],
                         fs[gi][1], fs[gi][2]);
    }
    // their plane sums
#pragma unroll
    for (int gi = 0; gi < 2; gi++) {
        const int w3 = wave_add32(fs[gi][0]), w4 = wave_add32(fs[gi][1]), w5 = wave_add32(fs[gi][2]);
        if (lane == 0) { int* q = rLS + 6 * wave + 3 * gi; q[0] = w3; q[1] = w4; q[2] = w5; }
    }
    __syncthreads();
    if (tid < 2 && (tid == 0 || two)) {
        const int gi = tid;
        int SXh = 0, SXl = 0, N32 = 0;
        for (int w = 0; w < NW; w++) { const int* q = rLS + 6 * w + 3 * gi; SXh += q[0]; SXl += q[1]; N32 += q[2]; }
        int* ri = (gi ? a.rowinfo2 : a.rowinfo1) + (size_t)r * 8;
        ri[0] = -16 + shg[gi]; ri[1] = 0; ri[2] = 0; ri[3] = 0; ri[4] = SXh; ri[5] = SXl; ri[6] = N32;
        i64* rex = gi ? a.rex2 : a.rex1;
        if (rec && rex) { rex[0] = -16 + shg[gi]; rex[1] = 0; }
    }
}

// The race over each stream's per-tile bests (base2.py:34-40, 114): one block per stream; block 0 writes the next
// position into the other position slot (read by the next step only, so no block waits for the others).  At a
// prompt position whose word is known only the position moves.
struct RaceArgs {
    const i64* part_v; const int* part_i; int nblk;
    int* seq; int seq_stride; int* words; int words_stride;
    const int* pos; const int* plen; int* nwords;
    int* pos_next;          // the other position slot: the next step reads it, no block of this launch does
};
__global__ __launch_bounds__(256) void k_race_rows(RaceArgs a) {
    __shared__ i64 bvs[4];
    __shared__ int bis[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = blockIdx.x;
    const int p = *a.pos;
    const bool skip = p < *a.plen - 1;
    if (!skip) {
        i64 bv = 0; int bi = -1;
        for (int g = tid; g < a.nblk; g += 256) {
            const i64 v = a.part_v[(size_t)r * a.nblk + g];
            const int ci = a.part_i[(size_t)r * a.nblk + g];
            if (ci >= 0 && (bi < 0 || v > bv || (v == bv && ci < bi))) { bv = v; bi = ci; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const i64 ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (lane == 0) { bvs[wave] = bv; bis[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            bv = bvs[0]; bi = bis[0];
            for (int w = 1; w < 4; w++)
                if (bis[w] >= 0 && (bi < 0 || bvs[w] > bv || (bvs[w] == bv && bis[w] < bi))) { bv = bvs[w]; bi = bis[w]; }
            a.seq[(size_t)r * a.seq_stride + p + 1] = bi;
            const int n = p + 1 - *a.plen;
            if (n >= 0) a.words[(size_t)r * a.words_stride + n] = bi;
        }
    }
    if (r == 0 && tid == 0) {
        *a.nwords = p + 1 - *a.plen + 1;
        *a.pos_next = p + 1;
    }
}

// The piles of a K-sliced bank whose blocks formed their light themselves (the stage product's finisher): the
// slices' accumulators and plane sums with the column sums, by the pile identity at the top of this file.
template <int KSP>
__global__ __launch_bounds__(256) void k_part_piles(GemmArgs a) {
    const int r = blockIdx.y;
    int ri[8];
    slice_facts<KSP>(a.sfacts, a.rows, r, ri);
    for (int j = blockIdx.x * 256 + threadIdx.x; j < a.N; j += gridDim.x * 256) {
        i64 ps = 0;                                  // (as the machine's finishers sum them)
#pragma unroll
        for (int q = 0; q < KSP; q++) ps += a.part[((size_t)q * a.rows + r) * a.N + j];
        a.Y[(size_t)r * a.ystride + j] = ps + 32768 * ((i64)ri[4] + a.csum[2 * j]) + 128 * ((i64)ri[5] + a.csum[2 * j + 1]) +
                                         16384 * (i64)a.K + 128 * (i64)ri[6];
    }
}

#define BINST_L(K, PRO, KSP) template __global__ void k_light<K, PRO, (K) / 4, KSP>(LightArgs);
BINST_L(768, PRO_EMBED, 1)
BINST_L(768, PRO_RACE_EMBED, 1)
BINST_L(768, PRO_GAUGE, 1)
BINST_L(768, PRO_TO16, 1)
BINST_L(3072, PRO_TO16, 1)
BINST_L(768, PRO_X16, 1)
BINST_L(3072, PRO_X16, 1)
BINST_L(768, PRO_ADD_GAUGE, 4)
template __global__ void k_py_rows<PY_EMBED>(PyRowArgs);
template __global__ void k_py_rows<PY_RACE_EMBED>(PyRowArgs);
template __global__ void k_py_rows<PY_ADD>(PyRowArgs);
template __global__ void k_py_rows<PY_GAUGE>(PyRowArgs);
#define BINST_G(K, NB, KSPLIT, EPI) template __global__ void k_gemm<K, NB, KSPLIT, EPI>(GemmArgs);
#define BINST_GR(RT) BINST_G(768, RT, 1, EPI_GAUGED) BINST_G(768, RT, 1, EPI_GAUGED_EDGE) BINST_G(768, RT, 1, EPI_PLAIN_ADD) \
    BINST_G(768, RT, 1, EPI_PART) BINST_G(768, RT, 1, EPI_PLAIN_EDGE) BINST_G(3072, RT, 4, EPI_PART) \
    BINST_G(768, RT, 1, EPI_PILE) BINST_G(3072, RT, 1, EPI_PILE) BINST_G(768, RT, 1, EPI_PLAIN)
BINST_GR(1)
template __global__ void k_gemm<768, 1, 1, EPI_PILE, 12>(GemmArgs);
template __global__ void k_part_piles<4>(GemmArgs);
#define BINST_H(RT) template __global__ void k_head_rows<RT, EPI_HEAD>(GemmArgs); \
    template __global__ void k_head_rows<RT, EPI_PILE>(GemmArgs); template __global__ void k_head_rows<RT, EPI_PHEAD>(GemmArgs);
BINST_H(1)
BINST_H(2)
BINST_H(3)
BINST_H(4)
