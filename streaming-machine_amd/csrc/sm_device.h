// Device-side integer arithmetic of the base-2 machine, with numpy's int64 semantics (base2.py is the spec):
// sums and products wrap modulo 2^64, a left shift by >= 64 gives 0, an arithmetic right shift by >= 64 gives
// 0 or -1.  Every function here is a restatement of the base2.py line it cites.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef long long i64;
typedef unsigned long long u64;

#define SMD __device__ __forceinline__

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

// base2.py:18-22  rshift(X, s): X * 2^-s rounded half up (s <= 0: a left shift)
SMD i64 rsh(i64 x, i64 s) {
    if (s <= 0) return shl(x, -s);
    return sar(wadd(x, shl(1, s - 1)), s);
}

// base2.py:42-48  log2fix(v): top-1 position t plus the table value of the next 16 bits (truncated)
SMD i64 log2fix(i64 v, const int* __restrict__ LOG2) {
    int t = bitlen_py(v) - 1;
    i64 m = t >= 16 ? (sar(v, t - 16) & 0xFFFF) : (shl(v, 16 - t) & 0xFFFF);
    return wadd((i64)t * 65536, (i64)LOG2[m]);
}

// base2.py:50-53  power(X, F) = rshift(X * EXP2[F & 0xFFFF], 16 - (F >> 16))
SMD i64 power(i64 x, i64 F, const int* __restrict__ EXP2) {
    i64 I = F >> 16, f = F & 0xFFFF;
    return rsh(wmul(x, (i64)EXP2[f]), wsub(16, I));
}

// base2.py:78-83  edge(H): the GELU share from PHI at rshift(H, 4) + 32768, then rshift(H * share, 16)
SMD i64 edge1(i64 h, const int* __restrict__ PHI) {
    i64 idx = wadd(rsh(h, 4), 32768);
    i64 share = idx < 0 ? 0 : (idx > 65535 ? 65536 : (i64)PHI[idx]);
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
SMD i64 gauge_ls(i64 s1, i64 s2, i64 ex, i64 log768, i64 eps40, const int* __restrict__ LOG2) {
    i64 V = wadd(wsub(wmul(768, s2), wmul(s1, s1)), eps_term(eps40, ex));
    return wadd(wsub(log2fix(V, LOG2) >> 1, log768), wmul(ex, 65536));
}

// ---------------- 64-wide wavefront reductions ----------------
SMD i64 wave_sum64(i64 v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
SMD i64 wave_or64(i64 v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}
SMD i64 wave_max64(i64 v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { i64 w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
    return v;
}

// sdot2: acc + a.lo * b.lo + a.hi * b.hi for packed int16 pairs (no clamp: callers bound the sums)
SMD int dot2(int a, int b, int acc) {
    typedef short short2v __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, a), __builtin_bit_cast(short2v, b), acc, false);
}
