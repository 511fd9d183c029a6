// Device-side integer arithmetic of the base-2 machine, with numpy's int64 semantics (base2.py is the spec):
// sums and products wrap modulo 2^64, a left shift by >= 64 gives 0, an arithmetic right shift by >= 64 gives
// 0 or -1.  Every function here is a restatement of the base2.py line it cites.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef long long i64;
typedef unsigned long long u64;

#define SMD __device__ __forceinline__

// The machine's four tables (base2_convert.py:48-61), read from memory.  (Recomputing an entry from its formula in
// float64 on the device measured slower than the read everywhere it was tried: the gauge's once-a-row entries, the
// edge's, the arrivals'.  The formulas below serve only the create-time check that the loaded tables are the
// reference's.)
struct Tables {
    const int* LOG2; const int* EXP2; const int* PHI; const int* ARR;
    int alen; i64 log768; i64 eps40;
    // derived, exact integer compositions of the tables above (built on the host at create):
    //   GPOW[r * 65536 + m] = EXP2[(log768 - ((r 65536 + LOG2[m]) >> 1)) & 0xFFFF]   the gauge's power factor
    //   HPOW[m]             = EXP2[(-LOG2[m]) & 0xFFFF]                              the arrivals' divisor
    //   PGPOW[r * 65536 + m] = EXP2[(-((r 65536 + LOG2[m]) >> 1)) & 0xFFFF]           Pythia's gauge factor
    // so that log2fix's mantissa m gives LOG2[m] and the EXP2 factor in two independent reads
    const int* GPOW; const int* HPOW; const int* PGPOW;
};

SMD i64 wadd(i64 a, i64 b) { return (i64)((u64)a + (u64)b); }
SMD i64 wsub(i64 a, i64 b) { return (i64)((u64)a - (u64)b); }
SMD i64 wmul(i64 a, i64 b) { return (i64)((u64)a * (u64)b); }
SMD i64 shl(i64 x, i64 n) { return ((u64)n >= 64) ? 0 : (i64)((u64)x << n); }
SMD i64 sar(i64 x, i64 n) { return ((u64)n >= 64) ? (x < 0 ? -1 : 0) : (x >> n); }
SMD int bitlen_u(u64 a) { return a ? 64 - __clzll((long long)a) : 0; }
// Python's int(v).bit_length() for an int64 value: the bit length of |v|
SMD int bitlen_py(i64 v) { return bitlen_u(v < 0 ? (u64)0 - (u64)v : (u64)v); }
// np.abs on int64 (INT64_MIN stays INT64_MIN)
SMD i64 iabs64(i64 v) { return v < 0 ? (i64)((u64)0 - (u64)v) : v; }
// foundation0/pythia_base2.py:63: the Pythia reference's rshift asserts |X| < 2^(62 + s) before a left shift
// (s < 0).  Checked here element by element (the reference checks an array's largest |X| against its most
// negative s, so it can stop where an element-wise check does not).
SMD bool pyshift_fails(i64 x, i64 s) {
    return s < 0 && (s < -62 ? x != 0 : (u64)iabs64(x) >= ((u64)1 << (62 + s)));
}

// ---- the tables' defining formulas, term for term as base2_convert.py:49-59 evaluates them (round half even);
// the create-time check compares every loaded entry with them
SMD int log2_entry(int m) { return (int)rint(log2(1.0 + (double)m / 65536.0) * 65536.0); }
SMD int exp2_entry(int f) { return (int)rint(pow(2.0, (double)f / 65536.0) * 65536.0); }
SMD int phi_entry(int i) { return (int)rint(0.5 * (1.0 + erf(((double)(i - 32768) / 4096.0) / 1.4142135623730951)) * 65536.0); }
SMD int arr_entry(i64 d) { return (int)rint(exp(-(double)d / 1024.0) * 16777216.0); }

SMD i64 tab_log2(const Tables& tb, i64 m) { return tb.LOG2[m]; }
SMD i64 tab_exp2(const Tables& tb, i64 f) { return tb.EXP2[f]; }
SMD i64 tab_phi(const Tables& tb, i64 i) { return tb.PHI[i]; }
// the arrival: 0 past the table (base2.py:97)
SMD int tab_arr(const Tables& tb, i64 d) { return d < tb.alen ? tb.ARR[d] : 0; }
// ARRF: the entry computed from its defining formula (arr_entry) instead of read, for a machine whose tables the
// create-time device check found equal to their formulas entry for entry, the arrival's alen + 1 included (so the
// two agree at every d >= 0): no dependent table read in the attention's chain.  Measured (same box, alternating):
// the batch-1 step 0.2480-0.2482 against 0.2484-0.2488 ms, Pythia at 32 streams 0.4025-0.4031 against
// 0.4055-0.4059; GPT-2 at 64 streams slower (0.5648-0.5662 against 0.5617-0.5622), so its attention reads the table
template <int ARRF>
SMD int arrival(const Tables& tb, i64 d) {
    if constexpr (ARRF) return d < tb.alen ? arr_entry(d) : 0;
    else return tab_arr(tb, d);
}

// base2.py:18-22  rshift(X, s): X * 2^-s rounded half up (s <= 0: a left shift)
SMD i64 rsh(i64 x, i64 s) {
    if (s <= 0) return shl(x, -s);
    return sar(wadd(x, shl(1, s - 1)), s);
}

// base2.py:42-48  log2fix(v): top-1 position t plus the table value of the next 16 bits (truncated)
SMD i64 log2fix(i64 v, const Tables& tb) {
    int t = bitlen_py(v) - 1;
    i64 m = t >= 16 ? (sar(v, t - 16) & 0xFFFF) : (shl(v, 16 - t) & 0xFFFF);
    return wadd((i64)t * 65536, tab_log2(tb, m));
}

// log2fix split into its top-1 position t and its mantissa index m (log2fix = t 65536 + LOG2[m])
SMD void log2_parts(i64 v, int& t, i64& m) {
    t = bitlen_py(v) - 1;
    m = t >= 16 ? (sar(v, t - 16) & 0xFFFF) : (shl(v, 16 - t) & 0xFFFF);
}
// The same reads at a wave-uniform index, two ways.
//   VEC = false: scalar loads (constant address space), counted apart from the vector loads, so they never wait
//   behind tiles still in flight; but they share their wait counter with LDS reads, so the next LDS read waits
//   for them too.
//   VEC = true: vector (buffer) loads of one address: in order behind the vector loads issued before them, and
//   waited for only where their value is used, so LDS reads in between (a GEMV phase's product reading its light)
//   do not wait for them.
// Measured at batch 1: the GEMV phases' gauge 1.4 % faster a step as vector loads; the one-wave attention's
// divisor slower (its value sum is short, so the vector loads' latency shows at the end): it stays scalar.
typedef const __attribute__((address_space(4))) int* cint_p;
template <bool VEC>
SMD i64 utab(const int* t, unsigned entries, int i) {
    i = __builtin_amdgcn_readfirstlane(i);
    if constexpr (VEC)
        return (int)__builtin_amdgcn_raw_buffer_load_b32(__builtin_amdgcn_make_buffer_rsrc(const_cast<int*>(t), 0,
                                                         (int)(entries * 4u), 0x00020000), i * 4, 0, 0);
    else
        return ((cint_p)t)[i];
}
template <bool VEC = false> SMD i64 utab_log2(const Tables& tb, int m) { return utab<VEC>(tb.LOG2, 65536u, m); }
template <bool VEC = false> SMD i64 utab_gpow(const Tables& tb, int r, int m) { return utab<VEC>(tb.GPOW, 131072u, r * 65536 + m); }
template <bool VEC = false> SMD i64 utab_pgpow(const Tables& tb, int r, int m) { return utab<VEC>(tb.PGPOW, 131072u, r * 65536 + m); }
SMD i64 utab_hpow(const Tables& tb, int m) { return utab<false>(tb.HPOW, 65536u, m); }
SMD i64 tab_gpow(const Tables& tb, int r, i64 m) { return tb.GPOW[r * 65536 + m]; }
SMD i64 tab_hpow(const Tables& tb, i64 m) { return tb.HPOW[m]; }

// base2.py:50-53  power(X, F) = rshift(X * EXP2[F & 0xFFFF], 16 - (F >> 16))
SMD i64 power(i64 x, i64 F, const Tables& tb) {
    i64 I = F >> 16, f = F & 0xFFFF;
    return rsh(wmul(x, tab_exp2(tb, f)), wsub(16, I));
}
// power(x, F) where EXP2[F & 0xFFFF] = e is known to the caller: for a gauged column F = (we + ex + 16) 65536 - LS,
// so F & 0xFFFF = (-LS) & 0xFFFF is the row's fine part whatever the column (base2.py:70)
SMD i64 power_known(i64 x, i64 F, i64 e) { return rsh(wmul(x, e), wsub(16, F >> 16)); }
// the same with EXP2[F & 0xFFFF] already at hand (e = the table value for fine part fe)
SMD i64 power_e(i64 x, i64 F, i64 fe, i64 e, const Tables& tb) {
    i64 I = F >> 16, f = F & 0xFFFF;
    return rsh(wmul(x, f == fe ? e : tab_exp2(tb, f)), wsub(16, I));
}

// base2.py:78-83  edge(H): the GELU share from PHI at rshift(H, 4) + 32768, then rshift(H * share, 16)
SMD i64 edge1(i64 h, const Tables& tb) {
    i64 idx = wadd(rsh(h, 4), 32768);
    i64 share = idx < 0 ? 0 : (idx > 65535 ? 65536 : tab_phi(tb, idx));
    return rsh(wmul(h, share), 16);
}

// base2.py:24-27  the water level: sh = max(bitlen(OR |x|) - 15, 0) from the OR of a row's magnitudes
SMD int water_shift(i64 orr) {
    int top = bitlen_py(orr);
    return top > 15 ? top - 15 : 0;
}

// base2.py:59  the eps term of the gauge: EPS40 >> (40 + 2 ex) (Python ints; the shift is >= 8 since ex >= -16)
SMD i64 eps_term(i64 eps40, i64 ex) {
    i64 es = 40 + 2 * ex;
    if (es >= 0) return es >= 63 ? 0 : (eps40 >> es);
    return shl(eps40, -es);
}

// base2.py:58-60  LS from S1, S2 (d = 768 values) and ex
SMD i64 gauge_ls(i64 s1, i64 s2, i64 ex, const Tables& tb) {
    i64 V = wadd(wsub(wmul(768, s2), wmul(s1, s1)), eps_term(tb.eps40, ex));
    return wadd(wsub(log2fix(V, tb) >> 1, tb.log768), wmul(ex, 65536));
}
// foundation0/pythia_base2.py:108-109  Pythia's gauge level LS = log2fix(V) >> 1 (no log2(d), no ex term: the
// centred lane is d x - S1, not x - S1 / d) and EXP2[(-LS) & 0xFFFF], its power factor for every lane
SMD i64 pgauge_ls_pow(i64 s1, i64 s2, i64 ex, const Tables& tb, i64& e2) {
    i64 V = wadd(wsub(wmul(768, s2), wmul(s1, s1)), eps_term(tb.eps40, ex));
    int t; i64 m;
    log2_parts(V, t, m);
    const i64 lg = utab_log2<true>(tb, (int)m);
    e2 = utab_pgpow<true>(tb, t & 1, (int)m);
    return wadd((i64)t * 65536, lg) >> 1;
}
// the same, also giving EXP2[(-LS) & 0xFFFF] (the power factor every gauged column uses) from one derived read
// (VEC: the table reads as vector loads, see utab)
template <bool VEC = false>
SMD i64 gauge_ls_pow(i64 s1, i64 s2, i64 ex, const Tables& tb, i64& e2) {
    i64 V = wadd(wsub(wmul(768, s2), wmul(s1, s1)), eps_term(tb.eps40, ex));
    int t; i64 m;
    log2_parts(V, t, m);
    const i64 lg = utab_log2<VEC>(tb, (int)m);      // V is the same in every lane: one address
    e2 = utab_gpow<VEC>(tb, t & 1, (int)m);
    const i64 l2 = wadd((i64)t * 65536, lg);
    return wadd(wsub(l2 >> 1, tb.log768), wmul(ex, 65536));
}
// the same at a row that differs between lanes (vector table reads)
SMD i64 gauge_ls_pow_v(i64 s1, i64 s2, i64 ex, const Tables& tb, i64& e2) {
    i64 V = wadd(wsub(wmul(768, s2), wmul(s1, s1)), eps_term(tb.eps40, ex));
    int t; i64 m;
    log2_parts(V, t, m);
    const i64 lg = tb.LOG2[m];
    e2 = tab_gpow(tb, t & 1, m);
    const i64 l2 = wadd((i64)t * 65536, lg);
    return wadd(wsub(l2 >> 1, tb.log768), wmul(ex, 65536));
}

// ---------------- bounded loads ----------------
typedef int v4i __attribute__((ext_vector_type(4)));
// A buffer resource over [base, base + bytes) (raw, stride 0; the gfx9 word-3 format): a load past the end
// returns zeros and sends no request to memory, so a fixed sequence of loads can cover a variable number of
// rows with no branch around them (a branch would make the next wait count every load in flight).
SMD __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
SMD v4i buf_load4(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
SMD int buf_load1(__amdgpu_buffer_rsrc_t r, unsigned off) { return (int)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0); }
SMD i64 buf_load8(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return (i64)__builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

// ---------------- wave64 reductions through DPP (a few VALU cycles per step) ----------------
// update_dpp(old = 0, ...): lanes a step does not reach contribute 0, the identity of +, | and max of naturals
#define DPP(v, ctrl, rm, bm) __builtin_amdgcn_update_dpp(0, (v), (ctrl), (rm), (bm), false)
// full wave reduction of a 32-bit value (+ or |), the total read from lane 63 into a uniform register
SMD int wave_add32(int v) {
    v += DPP(v, 0x111, 0xf, 0xf); v += DPP(v, 0x112, 0xf, 0xf); v += DPP(v, 0x114, 0xf, 0xe);
    v += DPP(v, 0x118, 0xf, 0xc); v += DPP(v, 0x142, 0xa, 0xf); v += DPP(v, 0x143, 0xc, 0xf);
    return __builtin_amdgcn_readlane(v, 63);
}
SMD unsigned wave_or32(unsigned u) {
    int v = (int)u;
    v |= DPP(v, 0x111, 0xf, 0xf); v |= DPP(v, 0x112, 0xf, 0xf); v |= DPP(v, 0x114, 0xf, 0xe);
    v |= DPP(v, 0x118, 0xf, 0xc); v |= DPP(v, 0x142, 0xa, 0xf); v |= DPP(v, 0x143, 0xc, 0xf);
    return (unsigned)__builtin_amdgcn_readlane(v, 63);
}
// 64-bit value moved by one DPP row shift (lo and hi words separately)
template <int CTRL, int BM>
SMD i64 dpp_shr64(i64 v) {
    const int lo = DPP((int)v, CTRL, 0xf, BM), hi = DPP((int)(v >> 32), CTRL, 0xf, BM);
    return (i64)(((u64)(unsigned)hi << 32) | (unsigned)lo);
}
// Sum of the lanes that share lane % TC (TC in 1, 2, 4, 8): in-row prefix steps of stride TC .. 8, then the
// four rows through two xor exchanges.  The totals end in lanes 16 - TC .. 15 of every row.
template <int TC>
SMD i64 wave_colsum64(i64 v) {
    if (TC <= 1) v += dpp_shr64<0x111, 0xf>(v);
    if (TC <= 2) v += dpp_shr64<0x112, 0xf>(v);
    if (TC <= 4) v += dpp_shr64<0x114, 0xe>(v);
    v += dpp_shr64<0x118, 0xc>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// ---------------- 64-wide wavefront reductions ----------------
struct OpOr { static constexpr i64 id = 0; SMD i64 operator()(i64 a, i64 b) const { return a | b; } };
struct OpAdd { static constexpr i64 id = 0; SMD i64 operator()(i64 a, i64 b) const { return (i64)((u64)a + (u64)b); } };
struct OpMax { static constexpr i64 id = INT64_MIN; SMD i64 operator()(i64 a, i64 b) const { return a > b ? a : b; } };
// a 64-bit value moved by one DPP step (both words by the same control); lanes the step does not write get id
template <int CTRL, int RM, int BM>
SMD i64 dpp64(i64 v, i64 id) {
    const int lo = __builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, RM, BM, false);
    const int hi = __builtin_amdgcn_update_dpp((int)(id >> 32), (int)(v >> 32), CTRL, RM, BM, false);
    return (i64)(((u64)(unsigned)hi << 32) | (unsigned)lo);
}
// the whole wave's op-total of a 64-bit value (the wave_add32 pattern: row shifts, then the two row broadcasts),
// read from lane 63 into uniform registers
template <class F>
SMD i64 wave_reduce64(i64 v, F op) {
    constexpr i64 id = F::id;
    v = op(v, dpp64<0x111, 0xf, 0xf>(v, id)); v = op(v, dpp64<0x112, 0xf, 0xf>(v, id));
    v = op(v, dpp64<0x114, 0xf, 0xe>(v, id)); v = op(v, dpp64<0x118, 0xf, 0xc>(v, id));
    v = op(v, dpp64<0x142, 0xa, 0xf>(v, id)); v = op(v, dpp64<0x143, 0xc, 0xf>(v, id));
    const int lo = __builtin_amdgcn_readlane((int)v, 63), hi = __builtin_amdgcn_readlane((int)(v >> 32), 63);
    return (i64)(((u64)(unsigned)hi << 32) | (unsigned)lo);
}
SMD i64 wave_or64(i64 v) { return wave_reduce64(v, OpOr()); }

// sdot2: acc + a.lo * b.lo + a.hi * b.hi for packed int16 pairs (no clamp: callers bound the sums)
SMD int dot2(int a, int b, int acc) {
    typedef short short2v __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, a), __builtin_bit_cast(short2v, b), acc, false);
}
