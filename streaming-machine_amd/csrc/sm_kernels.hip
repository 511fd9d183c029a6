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
#include "sm_kernels.h"

#define NTHR 256
typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------------------
// block reductions (4 waves)
template <typename F>
SMD i64 block_reduce(i64 v, i64* red, F op, int tid) {
    // red: 4 slots; caller guarantees red is free on entry; returns the reduced value to all threads
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = op(v, (i64)__shfl_xor(v, o, 64));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    i64 r = op(op(red[0], red[1]), op(red[2], red[3]));
    __syncthreads();
    return r;
}
struct OpOr { SMD i64 operator()(i64 a, i64 b) const { return a | b; } };
struct OpAdd { SMD i64 operator()(i64 a, i64 b) const { return (i64)((u64)a + (u64)b); } };
struct OpMax { SMD i64 operator()(i64 a, i64 b) const { return a > b ? a : b; } };

// ---------------------------------------------------------------------------------------------------------
// Prologue: the light entering the plate.  Writes xh/xl (NIN shorts each) into LDS and returns ex, LS.
template <int NIN, int PRO>
SMD void prologue(const GemvArgs& a, int tid, short* xh_s, short* xl_s, i64* red, i64& ex_o, i64& ls_o, bool rec) {
    constexpr int PER = NIN / NTHR;
    i64 v[PER];
    if (PRO == PRO_EMBED) {
        const int p = *a.pos;
        const i64 tok = a.seq[p];
#pragma unroll
        for (int m = 0; m < PER; m++) {
            int i = tid + NTHR * m;
            v[m] = wadd(a.wte[tok * 768 + i], a.wpe[(i64)p * 768 + i]);
            if (blockIdx.x == 0) a.Rw[i] = v[m];
        }
    } else {
#pragma unroll
        for (int m = 0; m < PER; m++) v[m] = a.X[tid + NTHR * m];
    }
    int sh = 0;
    if (PRO != PRO_X16) {
        i64 o = 0;
#pragma unroll
        for (int m = 0; m < PER; m++) o |= iabs64(v[m]);
        o = block_reduce(o, red, OpOr(), tid);
        sh = water_shift(o);
    }
    const i64 ex = -16 + sh;
    i64 s1 = 0, s2 = 0;
#pragma unroll
    for (int m = 0; m < PER; m++) {
        int i = tid + NTHR * m;
        i64 x = PRO == PRO_X16 ? v[m] : rsh(v[m], sh);
        int xi = (int)x;
        xh_s[i] = (short)(xi >> 8);
        xl_s[i] = (short)(xi & 255);
        s1 += x;
        s2 += x * x;
        if (rec && a.rx16) a.rx16[i] = x;
    }
    i64 ls = 0;
    if (PRO == PRO_GAUGE || PRO == PRO_EMBED) {
        s1 = block_reduce(s1, red, OpAdd(), tid);
        s2 = block_reduce(s2, red, OpAdd(), tid);
        ls = gauge_ls(s1, s2, ex, a.tb.log768, a.tb.eps40, a.tb.LOG2);
    }
    if (rec && a.rexls && tid == 0) { a.rexls[0] = ex; a.rexls[1] = ls; }
    ex_o = ex;
    ls_o = ls;
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------
template <int NIN, int TC, int NL>
SMD void load_tile(v4i (&w)[NL], const int4* __restrict__ W, int tile, int tid) {
    constexpr int UNITS = TC * NIN / 8;
    const v4i* base = reinterpret_cast<const v4i*>(W) + (size_t)tile * UNITS;
#pragma unroll
    for (int m = 0; m < NL; m++) {
        int u = tid + NTHR * m;
        if (UNITS % NTHR == 0 || u < UNITS) w[m] = __builtin_nontemporal_load(base + u);
    }
}

template <int NIN, int TC, int NL>
SMD i64 tile_partial(const v4i (&w)[NL], const short* xh_s, const short* xl_s, int tid) {
    constexpr int UNITS = TC * NIN / 8;
    int ah = 0, al = 0;
#pragma unroll
    for (int m = 0; m < NL; m++) {
        int u = tid + NTHR * m;
        if (UNITS % NTHR == 0 || u < UNITS) {
            const int c = u / TC;
            const int4 xh = reinterpret_cast<const int4*>(xh_s)[c];
            const int4 xl = reinterpret_cast<const int4*>(xl_s)[c];
            const v4i ww = w[m];
            ah = dot2(ww.x, xh.x, ah); ah = dot2(ww.y, xh.y, ah); ah = dot2(ww.z, xh.z, ah); ah = dot2(ww.w, xh.w, ah);
            al = dot2(ww.x, xl.x, al); al = dot2(ww.y, xl.y, al); al = dot2(ww.z, xl.z, al); al = dot2(ww.w, xl.w, al);
        }
    }
    return (i64)ah * 256 + (i64)al;
}

// The phase kernel: prologue (light), product over this block's tiles, epilogue per column.
template <int NIN, int TC, int PRO, int EPI>
__global__ __launch_bounds__(NTHR) void k_gemv(GemvArgs a) {
    constexpr int UNITS = TC * NIN / 8;
    constexpr int NL = (UNITS + NTHR - 1) / NTHR;
    static_assert(NTHR % TC == 0 && 64 % TC == 0, "tile width");
    __shared__ __align__(16) short xh_s[NIN];
    __shared__ __align__(16) short xl_s[NIN];
    __shared__ i64 red[4];
    __shared__ i64 redp[4 * TC];
    __shared__ int redi[TC];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    bool skip = false;
    int p = 0;
    if (EPI == EPI_HEAD) {
        p = *a.pos;
        skip = p < *a.plen - 1;     // a prompt position whose next word is already known
    }
    const bool rec = a.rec_pos && *a.rec_pos == (EPI == EPI_HEAD ? p : (a.pos ? *a.pos : -2));

    i64 best_v = 0;
    int best_i = -1;
    if (!skip) {
        int tile = blockIdx.x;
        v4i wc[NL];
        if (tile < a.ntiles) load_tile<NIN, TC, NL>(wc, a.W, tile, tid);   // weights in flight during the prologue
        i64 ex, ls;
        prologue<NIN, PRO>(a, tid, xh_s, xl_s, red, ex, ls, rec && blockIdx.x == 0);
        for (; tile < a.ntiles; tile += gridDim.x) {
            v4i wn[NL];
            const int nt = tile + gridDim.x;
            if (nt < a.ntiles) load_tile<NIN, TC, NL>(wn, a.W, nt, tid);
            i64 part = tile_partial<NIN, TC, NL>(wc, xh_s, xl_s, tid);
#pragma unroll
            for (int o = TC; o < 64; o <<= 1) part += __shfl_xor(part, o, 64);
            if (lane < TC) redp[wave * TC + lane] = part;
            __syncthreads();
            if (tid < TC) {
                const int j = tile * TC + tid;
                if (j < a.nout) {
                    const i64 pile = redp[tid] + redp[TC + tid] + redp[2 * TC + tid] + redp[3 * TC + tid];
                    if (rec && a.rpile) a.rpile[j] = pile;
                    const i64 we = a.we[j];
                    if (EPI == EPI_PILE) {
                        a.Y[j] = pile;
                    } else if (EPI == EPI_PLAIN_ADD) {
                        const i64 r = wadd(a.Y[j], wadd(rsh(pile, -(we + ex + 16)), a.bias[j]));
                        a.Y[j] = r;
                        if (rec && a.rout) a.rout[j] = r;
                    } else {
                        i64 y = wadd(power(pile, wsub((we + ex + 16) * 65536, ls), a.tb.EXP2), a.bias[j]);
                        if (EPI == EPI_GAUGED_EDGE) y = edge1(y, a.tb.PHI);
                        if (EPI == EPI_HEAD) {
                            if (rec && a.rlogits) a.rlogits[j] = y;
                            if (best_i < 0 || y > best_v) { best_v = y; best_i = j; }   // j grows: ties keep the first
                        } else {
                            a.Y[j] = y;
                            if (rec && a.rout) a.rout[j] = y;
                        }
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < NL; m++) wc[m] = wn[m];
        }
    }
    if (EPI != EPI_HEAD) return;

    // ---- the race (base2.py:34-40, 114): largest logit, ties to the lowest word ----
    if (tid < TC) { redp[tid] = best_v; redi[tid] = best_i; }
    __syncthreads();
    if (tid == 0) {
        i64 bv = 0; int bi = -1;
        for (int t = 0; t < TC; t++) {
            const int ci = redi[t];
            if (ci >= 0 && (bi < 0 || redp[t] > bv || (redp[t] == bv && ci < bi))) { bv = redp[t]; bi = ci; }
        }
        a.part_v[blockIdx.x] = bv;
        a.part_i[blockIdx.x] = bi;
        __threadfence();
        const unsigned prev = atomicAdd(a.counter, 1u);
        redi[0] = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!redi[0]) return;
    // the last block: every partial is visible (fence before each arrival, fence after ours)
    __threadfence();
    if (!skip) {
        i64 bv = 0; int bi = -1;
        for (int g = tid; g < (int)gridDim.x; g += NTHR) {
            const i64 v = __hip_atomic_load(&a.part_v[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int ci = __hip_atomic_load(&a.part_i[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ci >= 0 && (bi < 0 || v > bv || (v == bv && ci < bi))) { bv = v; bi = ci; }
        }
        // block argmax with ties to the lowest index
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const i64 ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (lane == 0) { redp[wave] = bv; redi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            bv = redp[0]; bi = redi[0];
            for (int w = 1; w < 4; w++)
                if (redi[w] >= 0 && (bi < 0 || redp[w] > bv || (redp[w] == bv && redi[w] < bi))) { bv = redp[w]; bi = redi[w]; }
            a.seq_w[p + 1] = bi;                  // the word goes straight back in (base2_stream.swift:143-146)
            const int n = p + 1 - *a.plen;
            if (n >= 0) a.words[n] = bi;
            *a.nwords = n + 1;
        }
    }
    if (tid == 0) {
        *a.pos_w = p + 1;
        *a.counter = 0u;
    }
}

// ---------------------------------------------------------------------------------------------------------
// Attention for the newest position of each stream, one block per (head, stream) (base2.py:85-100).
//   1. the head's q, k through their own water level (base2.py:93); k16, ek and the raw v go to the cache
//   2. scores over every cached position s <= p: rshift(q16 . k16, -(eq + ek + 7))          (base2.py:94)
//   3. the clock starts at the maximum; arrivals ARR[max - sc] (0 past the table)            (base2.py:96-97)
//   4. num = sum a v, out = power(num, -log2fix(sum a))                                        (base2.py:98-99)
// The maximum is global over the row before any arrival is read (two passes over LDS), so it is exact for any
// context length; the scores live in LDS (8 B each) and the arrivals beside them (4 B each).
__global__ __launch_bounds__(NTHR) void k_attend(AttArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    i64* sc = reinterpret_cast<i64*>(smem);                 // [ctx]
    int* av = reinterpret_cast<int*>(sc + a.ctx);            // [ctx]
    __shared__ int q16s[64], k16s[64], vs[64];
    __shared__ i64 red[4];
    __shared__ i64 numr[4][64];
    __shared__ int eqs, eks;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, b = blockIdx.y;
    const int p = *a.pos;
    const i64* qkv = a.QKV + (size_t)b * 2304;
    int* K16 = a.K16 + (size_t)b * a.ctx * 768;
    int* EK = a.EK + (size_t)b * a.ctx * 12;
    int* V = a.V + (size_t)b * a.ctx * 768;
    const bool rec = b == 0 && a.rec_pos && *a.rec_pos == p;

    // the new position's own key and value are used from LDS below: this block never reads back what it wrote
    if (wave < 2) {
        const i64 x = qkv[wave * 768 + h * 64 + lane];
        const int sh = water_shift(wave_or64(iabs64(x)));
        const int x16 = (int)rsh(x, sh);
        if (wave == 0) {
            q16s[lane] = x16;
            if (lane == 0) eqs = -16 + sh;
        } else {
            k16s[lane] = x16;
            K16[(size_t)p * 768 + h * 64 + lane] = x16;
            if (lane == 0) { eks = -16 + sh; EK[(size_t)p * 12 + h] = -16 + sh; }
        }
    } else if (wave == 2) {
        const i64 x = qkv[1536 + h * 64 + lane];
        if (x < (i64)INT32_MIN || x > (i64)INT32_MAX) atomicOr(a.err, SM_ERR_V32);
        vs[lane] = (int)x;
        V[(size_t)p * 768 + h * 64 + lane] = (int)x;
    }
    __syncthreads();

    const i64 eq = eqs;
    i64 mx = INT64_MIN;
    for (int s = tid; s <= p; s += NTHR) {
        i64 dot = 0, ek;
        if (s < p) {
            const int4* kr = reinterpret_cast<const int4*>(K16 + (size_t)s * 768 + h * 64);
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const int4 k4 = kr[c];
                dot += (i64)q16s[4 * c] * k4.x + (i64)q16s[4 * c + 1] * k4.y + (i64)q16s[4 * c + 2] * k4.z + (i64)q16s[4 * c + 3] * k4.w;
            }
            ek = EK[(size_t)s * 12 + h];
        } else {
            for (int c = 0; c < 64; c++) dot += (i64)q16s[c] * k16s[c];
            ek = eks;
        }
        const i64 v = rsh(dot, -(eq + ek + 7));
        sc[s] = v;
        mx = v > mx ? v : mx;
    }
    mx = block_reduce(mx, red, OpMax(), tid);
    i64 z = 0;
    for (int s = tid; s <= p; s += NTHR) {
        const i64 d = wsub(mx, sc[s]);
        const int w = d < a.tb.alen ? a.tb.ARR[d] : 0;
        av[s] = w;
        z += w;
    }
    z = block_reduce(z, red, OpAdd(), tid);   // includes a barrier: av[] complete
    i64 num = 0;
    for (int s = wave; s <= p; s += 4) {
        const int w = av[s];
        if (w) num += (i64)w * (s < p ? V[(size_t)s * 768 + h * 64 + lane] : vs[lane]);
    }
    numr[wave][lane] = num;
    __syncthreads();
    if (wave == 0) {
        const i64 tot = numr[0][lane] + numr[1][lane] + numr[2][lane] + numr[3][lane];
        const i64 F = wsub(0, log2fix(z, a.tb.LOG2));
        const i64 o = power(tot, F, a.tb.EXP2);
        a.out[(size_t)b * 768 + h * 64 + lane] = o;
        if (rec) a.ratt[h * 64 + lane] = o;
    }
}

// ---------------------------------------------------------------------------------------------------------
// Stage kernels: base2.py's stage functions on device buffers (unit parity and microbenchmarks).
__global__ void k_stage_rshift(const i64* x, const i64* s, i64* out, i64 n) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = rsh(x[i], s[i]);
}
__global__ void k_stage_power(const i64* x, const i64* F, i64* out, i64 n, const int* EXP2) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = power(x[i], F[i], EXP2);
}
__global__ void k_stage_log2fix(const i64* v, i64* out, i64 n, const int* LOG2) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = log2fix(v[i], LOG2);
}
__global__ void k_stage_edge(const i64* h, i64* out, i64 n, const int* PHI) {
    const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = edge1(h[i], PHI);
}
// to16 per row (one block per row); gauge != 0 also gives LS for rows of 768 (base2.py:24-27, 55-60)
__global__ __launch_bounds__(NTHR) void k_stage_rows(const i64* X, int n, int gauge, i64* x16, i64* ex, i64* LS, Tables tb) {
    __shared__ i64 red[4];
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
        s1 = block_reduce(s1, red, OpAdd(), tid);
        s2 = block_reduce(s2, red, OpAdd(), tid);
        if (tid == 0) LS[blockIdx.x] = gauge_ls(s1, s2, e, tb.log768, tb.eps40, tb.LOG2);
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
// explicit instantiations used by the host
#define INST(NIN, TC, PRO, EPI) template __global__ void k_gemv<NIN, TC, PRO, EPI>(GemvArgs);
INST(768, 8, PRO_EMBED, EPI_GAUGED)
INST(768, 8, PRO_GAUGE, EPI_GAUGED)
INST(768, 2, PRO_TO16, EPI_PLAIN_ADD)
INST(768, 8, PRO_GAUGE, EPI_GAUGED_EDGE)
INST(3072, 2, PRO_TO16, EPI_PLAIN_ADD)
INST(768, 8, PRO_GAUGE, EPI_HEAD)
// stage/product test instantiations: raw piles of a given light
INST(768, 8, PRO_X16, EPI_PILE)
INST(768, 2, PRO_X16, EPI_PILE)
INST(3072, 2, PRO_X16, EPI_PILE)
INST(3072, 8, PRO_X16, EPI_PILE)
