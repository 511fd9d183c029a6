/*
 * Shared by the oracle's C restatements (base2_oracle.c, pythia_oracle.c): numpy's int64 arithmetic and the
 * stage functions both machines use.  TEST INFRASTRUCTURE ONLY (see base2_oracle.c).
 */
#pragma once
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_E_BOUND 1      /* a product reached 2^52 (base2.py:31's assert) */
#define ORC_E_ARG 2

typedef int64_t i64;
typedef uint64_t u64;

/* ---------------- numpy int64 arithmetic ---------------- */
static inline i64 wadd(i64 a, i64 b) { return (i64)((u64)a + (u64)b); }
static inline i64 wsub(i64 a, i64 b) { return (i64)((u64)a - (u64)b); }
static inline i64 wmul(i64 a, i64 b) { return (i64)((u64)a * (u64)b); }
static inline i64 shl(i64 x, i64 n) { return ((u64)n >= 64) ? 0 : (i64)((u64)x << n); }
static inline i64 sar(i64 x, i64 n) { return ((u64)n >= 64) ? (x < 0 ? -1 : 0) : (x >> n); }
static inline int bitlen_u(u64 a) { return a ? 64 - __builtin_clzll(a) : 0; }
/* Python int(v).bit_length() of a numpy int64 value: the length of |v| */
static inline int bitlen_py(i64 v) { return bitlen_u(v < 0 ? (u64)0 - (u64)v : (u64)v); }
static inline i64 iabs(i64 v) { return v < 0 ? (i64)((u64)0 - (u64)v) : v; }   /* np.abs wraps at INT64_MIN */


/* stage functions defined in base2_oracle.c */
i64 orc_rshift1(i64 x, i64 s);
i64 orc_log2fix1(i64 v, const i64* LOG2);
i64 orc_power1(i64 x, i64 F, const i64* EXP2);
i64 orc_to16_row(const i64* x, i64 n, i64 e, i64* x16);
i64 orc_race(const i64* v, i64 n);
i64 orc_edge1(i64 h, const i64* PHI);
