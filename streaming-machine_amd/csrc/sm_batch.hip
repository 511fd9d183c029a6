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
    int* rowinfo;                 // [rows][8]: ex, LS lo, LS hi, e2, SXh, SXl, n32768
    Tables tb;
    const int* rec_pos; i64* rx16; i64* rexls;    // stream 0's record
};

struct GemmArgs {
    int K, N, rows, RT;
    const signed char* W;         // [N/16][KS][2][64][16]: wh, wl'
    const int* csum;              // [N][2]: SWh, SWl
    const int* we; const i64* bias;
    const signed char* planes; const int* rowinfo;
    i64* Y; int ystride;          // output rows [rows][ystride] (or the stream R for EPI_PLAIN_ADD)
    Tables tb;
    const int* pos; const int* plen;
    i64* part_v; int* part_i; int nblk;   // EPI_HEAD: per (row, block) best
    const int* rec_pos; i64* rpile; i64* rout; i64* rlogits;
};

// ---------------------------------------------------------------------------------------------------------
// One block (256 threads) per stream row: the light of base2.py:24-27 (and the gauge of :55-60), written as
// MFMA A planes plus the row's exponent, gauge, power factor and plane sums.
template <int K, int PRO>
__global__ __launch_bounds__(256) void k_light(LightArgs a) {
    constexpr int PER = K / 256, KS = K / 64;
    __shared__ int red[32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = blockIdx.x;
    const int p = a.pos ? *a.pos : 0;              // the stage product (PRO_X16) has no position
    if (a.skip_prompt && p < *a.plen - 1) return;
    i64 v[PER];
    if (PRO == PRO_EMBED) {
        const i64 tok = a.seq[(size_t)r * a.seq_stride + p];
#pragma unroll
        for (int m = 0; m < PER; m++) {
            const int i = tid + 256 * m;
            v[m] = wadd(a.wte[tok * 768 + i], a.wpe[(i64)p * 768 + i]);
            a.Rw[(size_t)r * 768 + i] = v[m];
        }
    } else {
#pragma unroll
        for (int m = 0; m < PER; m++) v[m] = a.X[(size_t)r * K + tid + 256 * m];
    }
    int sh = 0;                                     // PRO_X16: the lights are given
    if (PRO != PRO_X16) {
        u64 o = 0;
#pragma unroll
        for (int m = 0; m < PER; m++) o |= (u64)iabs64(v[m]);
        const unsigned olo = wave_or32((unsigned)o), ohi = wave_or32((unsigned)(o >> 32));
        if (lane == 0) { red[2 * wave] = (int)olo; red[2 * wave + 1] = (int)ohi; }
        __syncthreads();
        u64 all = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) all |= ((u64)(unsigned)red[2 * w + 1] << 32) | (unsigned)red[2 * w];
        sh = water_shift((i64)all);
    }
    const i64 ex = -16 + sh;
    const bool rec = r == 0 && a.rec_pos && *a.rec_pos == p;
    int s1 = 0, sxh = 0, sxl = 0, n32 = 0;
    i64 s2 = 0;
    signed char* pl = a.planes + (size_t)(r >> 4) * KS * 3 * 1024;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int k = tid + 256 * m;
        const int x = (int)rsh(v[m], sh);
        s1 += x;
        s2 += (i64)x * x;
        if (rec && a.rx16) a.rx16[k] = x;
        const int c = x == 32768;
        const int xc = x - c;                      // +32768 -> 32767, the rest unchanged
        const int xh = xc >> 8, xl = (xc & 255) - 128;
        sxh += xh; sxl += xl; n32 += c;
        const int s = k >> 6, kk = k & 63;
        const size_t off = (size_t)s * 3 * 1024 + (size_t)((r & 15) + 16 * (kk >> 4)) * 16 + (kk & 15);
        pl[off] = (signed char)xh;
        pl[off + 1024] = (signed char)xl;
        pl[off + 2048] = (signed char)c;
    }
    const int w1 = wave_add32(s1), w2h = wave_add32((int)(s2 >> 16)), w2l = wave_add32((int)(s2 & 0xFFFF));
    const int w3 = wave_add32(sxh), w4 = wave_add32(sxl), w5 = wave_add32(n32);
    if (lane == 0) { int* q = red + 8 + 6 * wave; q[0] = w1; q[1] = w2h; q[2] = w2l; q[3] = w3; q[4] = w4; q[5] = w5; }
    __syncthreads();
    if (tid == 0) {
        i64 S1 = 0, S2h = 0, S2l = 0, SXh = 0, SXl = 0, N32 = 0;
        for (int w = 0; w < 4; w++) {
            const int* q = red + 8 + 6 * w;
            S1 += q[0]; S2h += q[1]; S2l += q[2]; SXh += q[3]; SXl += q[4]; N32 += q[5];
        }
        i64 ls = 0, e2 = 0;
        if (PRO == PRO_GAUGE || PRO == PRO_EMBED) ls = gauge_ls_pow(S1, (S2h << 16) + S2l, ex, a.tb, e2);
        int* ri = a.rowinfo + (size_t)r * 8;
        ri[0] = (int)ex; ri[1] = (int)(u64)ls; ri[2] = (int)((u64)ls >> 32); ri[3] = (int)e2;
        ri[4] = (int)SXh; ri[5] = (int)SXl; ri[6] = (int)N32;
        if (rec && a.rexls) { a.rexls[0] = ex; a.rexls[1] = ls; }
    }
}

// ---------------------------------------------------------------------------------------------------------
// One block (4 waves) per 16-column tile; wave w takes the 64-k steps s = w, w + 4, .. (split K), every wave all
// RT row tiles; the four partial results meet in LDS and each (row, column) pile gets its epilogue.
template <int K, int RT, int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    constexpr int KS = K / 64;
    __shared__ i64 acc_s[4][RT * 16][16 + 1];          // per wave partial piles [row][col] (padded)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = blockIdx.x;                          // column tile
    const int p = a.pos ? *a.pos : 0;                   // the stage product (EPI_PILE) has no position
    if (EPI == EPI_HEAD && p < *a.plen - 1) return;    // a prompt position: the race kernel only advances
    // which row tiles need the +32768 correction (uniform)
    unsigned corr = 0;
    for (int rt = 0; rt < RT; rt++) {
        int n = 0;
        for (int i = 0; i < 16; i++) if (rt * 16 + i < a.rows) n += a.rowinfo[(size_t)(rt * 16 + i) * 8 + 6];
        if (n) corr |= 1u << rt;
    }
    v4i_b hh[RT], hl[RT], lh[RT], ll[RT], ch[RT], cl[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) hh[t] = hl[t] = lh[t] = ll[t] = ch[t] = cl[t] = v4i_b{0, 0, 0, 0};
    const v4i_b* Wp = reinterpret_cast<const v4i_b*>(a.W) + (size_t)nt * KS * 2 * 64 + lane;
    const v4i_b* Ap = reinterpret_cast<const v4i_b*>(a.planes) + lane;
    for (int s = wave; s < KS; s += 4) {
        const v4i_b wh = __builtin_nontemporal_load(Wp + (size_t)s * 128);
        const v4i_b wl = __builtin_nontemporal_load(Wp + (size_t)s * 128 + 64);
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const v4i_b* ap = Ap + ((size_t)t * KS + s) * 3 * 64;
            const v4i_b xh = ap[0], xl = ap[64];
            hh[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh, wh, hh[t], 0, 0, 0);
            hl[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xh, wl, hl[t], 0, 0, 0);
            lh[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl, wh, lh[t], 0, 0, 0);
            ll[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xl, wl, ll[t], 0, 0, 0);
            if (corr & (1u << t)) {
                const v4i_b c = ap[128];
                ch[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c, wh, ch[t], 0, 0, 0);
                cl[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c, wl, cl[t], 0, 0, 0);
            }
        }
    }
    // this wave's partial piles (the plane-sum terms are added once, below)
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = t * 16 + 4 * (lane >> 4) + q, col = lane & 15;
            acc_s[wave][row][col] = 65536 * (i64)hh[t][q] + 256 * ((i64)hl[t][q] + lh[t][q]) + ll[t][q] +
                                    256 * (i64)ch[t][q] + cl[t][q];
        }
    __syncthreads();
    const bool rec0 = a.rec_pos && *a.rec_pos == p;
    for (int e = tid; e < RT * 256; e += 256) {
        const int row = e >> 4, col = e & 15, j = nt * 16 + col;
        if (row >= a.rows || j >= a.N) continue;
        const int* ri = a.rowinfo + (size_t)row * 8;
        const i64 ex = ri[0];
        const i64 ls = (i64)(((u64)(unsigned)ri[2] << 32) | (unsigned)ri[1]);
        const i64 e2 = ri[3];
        const i64 pile = acc_s[0][row][col] + acc_s[1][row][col] + acc_s[2][row][col] + acc_s[3][row][col] +
                         32768 * ((i64)ri[4] + a.csum[2 * j]) + 128 * ((i64)ri[5] + a.csum[2 * j + 1]) +
                         16384 * (i64)K + 128 * (i64)ri[6];
        const bool rec = rec0 && row == 0;
        if (rec && a.rpile) a.rpile[j] = pile;
        const i64 we = a.we[j], bc = a.bias[j];
        if (EPI == EPI_PILE) {
            a.Y[(size_t)row * a.ystride + j] = pile;
        } else if (EPI == EPI_PLAIN_ADD) {
            i64* y = a.Y + (size_t)row * a.ystride + j;
            const i64 r = wadd(*y, wadd(rsh(pile, -(we + ex + 16)), bc));
            *y = r;
            if (rec && a.rout) a.rout[j] = r;
        } else {
            const i64 fe = wsub(0, ls) & 0xFFFF;
            i64 y = wadd(power_e(pile, wsub(wmul(we + ex + 16, 65536), ls), fe, e2, a.tb), bc);
            if (EPI == EPI_GAUGED_EDGE) y = edge1(y, a.tb);
            if (EPI == EPI_HEAD) {
                if (rec && a.rlogits) a.rlogits[j] = y;
                acc_s[0][row][col] = y;               // only this thread reads or writes this cell
            } else {
                a.Y[(size_t)row * a.ystride + j] = y;
                if (rec && a.rout) a.rout[j] = y;
            }
        }
    }
    if (EPI != EPI_HEAD) return;
    __syncthreads();
    // per row: the largest logit of this tile, ties to the lowest column
    for (int row = tid; row < RT * 16; row += 256) {
        if (row >= a.rows) continue;
        i64 b = 0; int ib = -1;
        for (int col = 0; col < 16; col++) {
            const int j = nt * 16 + col;
            if (j >= a.N) break;
            const i64 y = acc_s[0][row][col];
            if (ib < 0 || y > b) { b = y; ib = j; }
        }
        a.part_v[(size_t)row * a.nblk + nt] = b;
        a.part_i[(size_t)row * a.nblk + nt] = ib;
    }
}

// The race over each stream's per-tile bests (base2.py:34-40, 114): one block per stream; the last block to
// finish advances the shared position.  At a prompt position whose word is known only the position moves.
struct RaceArgs {
    const i64* part_v; const int* part_i; int nblk;
    int* seq; int seq_stride; int* words; int words_stride;
    int* pos; const int* plen; int* nwords; unsigned* counter;
};
__global__ __launch_bounds__(256) void k_race_rows(RaceArgs a) {
    __shared__ i64 bvs[4];
    __shared__ int bis[4];
    __shared__ int last;
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
    if (tid == 0) {
        __threadfence();
        last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (last && tid == 0) {
        *a.nwords = p + 1 - *a.plen + 1;
        *a.pos = p + 1;
        *a.counter = 0u;
    }
}

#define BINST_L(K, PRO) template __global__ void k_light<K, PRO>(LightArgs);
BINST_L(768, PRO_EMBED)
BINST_L(768, PRO_GAUGE)
BINST_L(768, PRO_TO16)
BINST_L(3072, PRO_TO16)
BINST_L(768, PRO_X16)
BINST_L(3072, PRO_X16)
#define BINST_G(K, RT, EPI) template __global__ void k_gemm<K, RT, EPI>(GemmArgs);
#define BINST_GR(RT) BINST_G(768, RT, EPI_GAUGED) BINST_G(768, RT, EPI_PLAIN_ADD) BINST_G(768, RT, EPI_GAUGED_EDGE) \
    BINST_G(3072, RT, EPI_PLAIN_ADD) BINST_G(768, RT, EPI_HEAD) BINST_G(768, RT, EPI_PILE) BINST_G(3072, RT, EPI_PILE)
BINST_GR(1)
BINST_GR(2)
BINST_GR(3)
BINST_GR(4)
