// The batch-1 attention spread over the GPU: one new position's attention (base2.py:85-100 for the last row;
// foundation0/pythia_base2.py:125-141) with each head's cached positions cut into chunks of ACH_SPLIT, one block a
// (head, chunk), in three launches (the machine launches the first two, and proj's blocks then form the output row
// from the accumulators themselves: PRO_ATT / PRO_PATT in sm_kernels.hip; the stage entry point launches all three):
//   k_att_scores  the new q (and, in the chunk holding p, the new k and v into the cache) through their water
//                 levels (base2.py:93); the chunk's scores rshift(q16 . k16, -(eq + ek + 7)) (base2.py:94) into
//                 a score row, and the chunk's maximum; block (h, 0) empties the head's accumulator
//   k_att_mix     the head's maximum over the chunk maxima, the chunk's arrivals ARR[max - sc] (base2.py:96-97),
//                 their sum and the chunk's value sums sum a v (base2.py:98), added into the head's accumulator by
//                 64-bit atomics
//   k_att_finish  out = power(num, -log2fix(Z)) (base2.py:99) from the accumulator
// Exactness: every arrival is taken against the head's global maximum, which only exists once every chunk's
// scores are in (the kernel boundary between the first two launches); the value sums and the arrival sum are
// integer sums, so the chunks' partials add to the one-block kernel's totals in any order (two's-complement
// wrap, as numpy's int64).  The one-block kernel (k_attend) reads a head's cache on one CU, whose HBM rate
// (tens of GB/s) bounds it past a few hundred positions; here every CU holding a chunk reads 25 KB.
#define ACH_SPLIT 64   // positions a chunk: one pass of 256 threads, four lanes a position
#define ACC_W 68       // accumulator words a head: the 64 value sums, the arrival sum, the largest weighed |v|

// AttArgs fields used here beyond the one-block kernel's: asc [12][ctx] scores, acm [12][ncm] chunk maxima,
// aacc [12][ACC_W] accumulators (batch 1: stream 0's cache rows)
template <int MODEL>
__global__ __launch_bounds__(256) void k_att_scores(AttArgs a) {
    const int h = blockIdx.x, c = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sl = tid >> 2, qd = tid & 3;                  // position in the chunk, the lane's 16 dimensions
    __shared__ __align__(16) int q16s[64];
    __shared__ __align__(16) int k16s[64];
    __shared__ i64 red[4];
    __shared__ int eqs, eks;
    // the new q (wave 0), k (wave 1) and v (wave 2), requested before the position (vector loads complete in order)
    auto qkv_at = [&](int part) { return MODEL == 1 ? h * 192 + part * 64 + lane : part * 768 + h * 64 + lane; };
    i64 xnew = wave < 3 ? a.QKV[qkv_at(wave)] : 0;
    const int p = *a.pos;
    const int s0 = c * ACH_SPLIT;
    if (s0 > p) return;                                     // (uniform) a chunk past the position
    const bool mine = p - s0 < ACH_SPLIT;                   // this chunk holds the new position
    const size_t hb = (size_t)h * a.ctx;
    short* K16 = a.K16 + hb * 64;
    i64* KM = a.KM + hb;
    int* EK = a.EK + hb;
    int* V = a.V + hb * 64;
    // Pythia: the turn's cos and sin of dimension lane at position p (lanes past rot read zeros)
    int tcos = 0, tsin = 0;
    if constexpr (MODEL == 1) {
        const int r = a.rot >> 1, ti = lane < r ? lane : lane - r;
        const unsigned lim = (unsigned)((p + 1) * r) * 4u, off = (unsigned)(p * r + ti) * 4u;
        tcos = buf_load1(buf_rsrc(a.cosT, lim), off);
        tsin = buf_load1(buf_rsrc(a.sinT, lim), off);
    }
    // the chunk's cached keys, their levels and masks (bounded at p: rows from p on read zeros, no request)
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(K16, (unsigned)p * 128), re = buf_rsrc(EK, (unsigned)p * 4),
                                 rm = buf_rsrc(KM, (unsigned)p * 8);
    const unsigned s = (unsigned)(s0 + sl);
    const v4i k0 = buf_load4(rk, s * 128 + qd * 32), k1 = buf_load4(rk, s * 128 + qd * 32 + 16);
    const int ekc = buf_load1(re, s * 4);
    const i64 kmc = buf_load8(rm, s * 8);
    // the chunk's cached values, requested for k_att_mix's block of the same index (dispatched to the same XCD, so
    // the lines wait in its L2, and in the Infinity Cache either way): one dword a 128-byte line, threads 0-127;
    // the others' offset is past the resource (no request)
    const unsigned voff = tid < 128 ? (unsigned)s0 * 256u + (unsigned)tid * 128u : 0xFFFFFF00u;
    const int pfv = buf_load1(buf_rsrc(V, (unsigned)p * 256), voff);
    if constexpr (MODEL == 1) __builtin_amdgcn_sched_barrier(0);   // (the loads above stay issued here)
    if (MODEL == 1 && (wave == 0 || (wave == 1 && mine))) {        // the turns (pythia_base2.py:116-123)
        const int r = a.rot >> 1;
        const i64 partner = __shfl(xnew, lane < r ? lane + r : lane - r, 64);
        if (lane < a.rot) {
            if (iabs64(xnew) >= ((i64)1 << 31)) atomicOr(a.err, SM_ERR_RANGE);
            xnew = turn1<0>(xnew, partner, lane < r, tcos, tsin, 0.0, 0.0);
        }
    }
    if (wave == 0 || (wave == 1 && mine)) {
        const int sh = water_shift(wave_or64(iabs64(xnew)));
        const int x16 = (int)rsh(xnew, sh);
        if (wave == 0) {
            q16s[lane] = x16;
            if (lane == 0) eqs = -16 + sh;
        } else {
            k16s[lane] = x16;
            key_store(K16 + (size_t)p * 64, KM + p, x16, lane);
            if (lane == 0) {
                eks = -16 + sh;
                EK[p] = -16 + sh;
            }
        }
    } else if (wave == 2 && mine) {
        v_store(a, (size_t)h, p, lane, xnew);
    }
    __syncthreads();
    // the chunk's scores (base2.py:94 / pythia_base2.py:135)
    const i64 eq = eqs;
    v4i qv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) qv[u] = reinterpret_cast<const v4i*>(q16s)[4 * qd + u];
    i64 dot = 0, ek = ekc;
    if ((int)s < p) {
        const v4i kk[2] = {k0, k1};
        dot = dot16(qv, kk) + dot16_mask(qv, (unsigned)((u64)kmc >> (16 * qd)) & 0xFFFFu);
    } else if ((int)s == p) {                               // the new key (int32, from LDS)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const v4i kn = reinterpret_cast<const v4i*>(k16s)[4 * qd + u];
            dot += (i64)qv[u].x * kn.x + (i64)qv[u].y * kn.y + (i64)qv[u].z * kn.z + (i64)qv[u].w * kn.w;
        }
        ek = eks;
    }
    dot += dpp64<0xB1, 0xf, 0xf>(dot, 0);                  // quad_perm [1, 0, 3, 2]: the position's four lanes
    dot += dpp64<0x4E, 0xf, 0xf>(dot, 0);                  // quad_perm [2, 3, 0, 1]
    i64 v = INT64_MIN;
    if ((int)s <= p) {
        v = MODEL == 1 ? rsh(wmul(dot, a.ehalf), wsub(16, wsub(wmul(eq + ek + 10, 65536), a.half) >> 16))
                       : rsh(dot, -(eq + ek + 7));
        if (qd == 0) a.asc[hb + s] = v;
    }
    const i64 mx = block_reduce<OpMax, 4>(v, red, OpMax(), tid);
    if (tid == 0) a.acm[(size_t)h * a.ncm + c] = mx;
    if (c == 0 && tid < ACC_W) a.aacc[(size_t)h * ACC_W + tid] = 0;
    asm volatile("" ::"v"(pfv));                            // (the value requests stay)
}

// ARRF: arrivals from their formula (the tables verified equal to it), as the one-block kernel takes them
template <int MODEL, int ARRF>
__global__ __launch_bounds__(256) void k_att_mix(AttArgs a) {
    const int h = blockIdx.x, c = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d4 = tid & 15, g = tid >> 4;                  // four dimensions, position group (16 a chunk pass)
    __shared__ __align__(16) int arr_s[ACH_SPLIT];
    __shared__ i64 red[4];
    __shared__ i64 numr[16][64];
    const int p = *a.pos;
    const int s0 = c * ACH_SPLIT;
    if (s0 > p) return;                                     // (uniform)
    const int nc = p / ACH_SPLIT + 1;                       // chunks holding positions 0..p
    const size_t hb = (size_t)h * a.ctx;
    // requests: the chunk maxima (thread t < nc its own), the chunk's scores (wave 0, lane = position), its values
    // (16 lanes a 256-byte row, positions s0 + g + 16 i), all bounded so that nothing past p is requested
    const i64 cmv = buf_load8(buf_rsrc(a.acm + (size_t)h * a.ncm, (unsigned)nc * 8u), (unsigned)tid * 8u);
    const i64 scv = buf_load8(buf_rsrc(a.asc + hb, (unsigned)(p + 1) * 8u), wave == 0 ? (unsigned)(s0 + lane) * 8u : 0xFFFFFF00u);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(a.V + hb * 64, (unsigned)(p + 1) * 256u);
    v4i vp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) vp[i] = buf_load4(rv, (unsigned)(s0 + g + 16 * i) * 256u + d4 * 16);
    const int vbg = vbig_load(a, (size_t)h);                // the head holds a value past 32 bits (read whole below)
    // the clock starts at the head's maximum (base2.py:96)
    const i64 M = block_reduce<OpMax, 4>(tid < nc ? cmv : INT64_MIN, red, OpMax(), tid);
    // arrivals (base2.py:96-97), wave 0 a position each, and their sum
    i64 z = 0;
    if (wave == 0) {
        const int w = s0 + lane <= p ? arrival<ARRF>(a.tb, wsub(M, scv)) : 0;
        arr_s[lane] = w;
        z = wave_reduce64((i64)w, OpAdd());
    }
    __syncthreads();
    // the chunk's value sums of dimensions 4 d4 .. + 3 (base2.py:98); positions past p weigh 0 (their values read 0)
    i64 n0 = 0, n1 = 0, n2 = 0, n3 = 0;
    int vmax = 0;                                           // Pythia: the largest |v| weighed (the 2^62 assert)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int w = arr_s[g + 16 * i];
        const v4i x = vp[i];
        n0 += (i64)w * x.x; n1 += (i64)w * x.y; n2 += (i64)w * x.z; n3 += (i64)w * x.w;
        if (MODEL == 1 && w) vmax = max(vmax, max(max(abs(x.x), abs(x.y)), max(abs(x.z), abs(x.w))));
    }
    i64 vm64 = vmax;
    if (a.V64 && __builtin_amdgcn_readfirstlane(vbg)) {     // (block-uniform) the head's values whole
        n0 = n1 = n2 = n3 = 0;
        vm64 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int sv = s0 + g + 16 * i;
            if (sv > p) break;
            const i64 w = arr_s[g + 16 * i];
            i64 x[4];
            for (int j = 0; j < 4; j++) x[j] = v_whole(a, hb, sv, 4 * d4 + j);
            n0 = wadd(n0, wmul(w, x[0])); n1 = wadd(n1, wmul(w, x[1])); n2 = wadd(n2, wmul(w, x[2])); n3 = wadd(n3, wmul(w, x[3]));
            if (MODEL == 1 && w) vm64 = max(max(vm64, max(iabs64(x[0]), iabs64(x[1]))), max(iabs64(x[2]), iabs64(x[3])));
        }
    }
    numr[g][4 * d4] = n0; numr[g][4 * d4 + 1] = n1; numr[g][4 * d4 + 2] = n2; numr[g][4 * d4 + 3] = n3;
    i64 vm = 0;
    if constexpr (MODEL == 1) vm = block_reduce<OpMax, 4>(vm64, red, OpMax(), tid);   // (its barriers publish numr)
    else __syncthreads();
    if (wave == 0) {
        i64 tot = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) tot = wadd(tot, numr[i][lane]);
        i64* acc = a.aacc + (size_t)h * ACC_W;
        atomicAdd(reinterpret_cast<unsigned long long*>(acc + lane), (unsigned long long)tot);
        if (lane == 0) {
            atomicAdd(reinterpret_cast<unsigned long long*>(acc + 64), (unsigned long long)z);
            if (MODEL == 1) atomicMax(reinterpret_cast<unsigned long long*>(acc + 65), (unsigned long long)vm);
        }
    }
}

// one block of 64 threads a head: out = power(num, -log2fix(Z)) (base2.py:99); Pythia: exact in 128 bits, with the
// reference's asserts (|v| sum(a) < 2^62, a result that fits; pythia_base2.py:139, 90)
template <int MODEL, int REC>
__global__ __launch_bounds__(64) void k_att_finish(AttArgs a) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const i64* acc = a.aacc + (size_t)h * ACC_W;
    const i64 tot = acc[lane], z = acc[64];
    int zt;
    i64 zm;
    log2_parts(z, zt, zm);
    const i64 F = wsub(0, wadd((i64)zt * 65536, utab_log2(a.tb, (int)zm)));   // -log2fix(Z), the same in every lane
    const i64 zhp = utab_hpow(a.tb, (int)zm);
    i64 o;
    if (MODEL == 1) {
        if ((double)acc[65] * (double)z >= 4611686018427387904.0) atomicOr(a.err, SM_ERR_RANGE);
        const __int128 X = (__int128)tot * zhp;
        const i64 sft = 16 - (F >> 16);
        const __int128 r = sft >= 100 ? (__int128)0 : (X + ((__int128)1 << (sft - 1))) >> sft;
        if (r > (__int128)INT64_MAX || r < (__int128)INT64_MIN) atomicOr(a.err, SM_ERR_RANGE);
        o = (i64)r;
    } else {
        o = power_e(tot, F, F & 0xFFFF, zhp, a.tb);
    }
    a.out[h * 64 + lane] = o;
    if (a.out32) a.out32[h * 64 + lane] = (int)o;
    if (a.out_or) {
        const i64 w = wave_or64(iabs64(o));
        if (lane == 0) a.out_or[h] = w;
    }
    if (REC && a.rec_pos && *a.rec_pos == *a.pos) a.ratt[h * 64 + lane] = o;
}

template __global__ void k_att_scores<0>(AttArgs);
template __global__ void k_att_scores<1>(AttArgs);
template __global__ void k_att_mix<0, 0>(AttArgs);
template __global__ void k_att_mix<0, 1>(AttArgs);
template __global__ void k_att_mix<1, 0>(AttArgs);
template __global__ void k_att_mix<1, 1>(AttArgs);
template __global__ void k_att_finish<0, 0>(AttArgs);
template __global__ void k_att_finish<0, 1>(AttArgs);
template __global__ void k_att_finish<1, 0>(AttArgs);
template __global__ void k_att_finish<1, 1>(AttArgs);
