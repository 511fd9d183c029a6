/*
 * sm_base2.h - C ABI of the MI355X integer ("all base 2") GPT-2 decode step.
 *
 * One shared library (libsm_base2.so, gfx950 HIP) owns the device weights, the tables and the per-layer
 * integer KV cache, and runs the decode step: every number a whole number, every emitted word the word
 * base2.py's forward() gives on the same inputs.  All entry points return 0 (SM_OK) or a negative code;
 * sm_last_error() gives the calling thread's last message.  No exception crosses this ABI.
 *
 * The reference has no C ABI: its machine is base2.py's stage functions (the operator API research code
 * wraps, e.g. recording/C_plain.py:15-22) and the Swift/Metal streaming machine (base2_stream.swift).  Each
 * declaration below names the reference interface it replaces.
 *
 * Threading: a machine is one HIP stream and is not thread-safe; callers serialise calls on a handle.
 */
#ifndef SM_BASE2_H
#define SM_BASE2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SM_OK = 0,
    SM_E_ARG = -1,       /* bad argument (sizes, ids, state) */
    SM_E_IO = -2,        /* a layout file is missing, short or malformed */
    SM_E_HIP = -3,       /* a HIP runtime call failed */
    SM_E_OOM = -4,       /* device allocation failed */
    SM_E_CTX = -5,       /* the context (positions) would pass max_ctx */
    SM_E_OVERFLOW = -6,  /* an integer left the range the device layout holds (checked on the device) */
    SM_E_STATE = -7      /* call out of order (e.g. generate before prefill) */
};

typedef struct sm_machine sm_machine;

typedef struct {
    int32_t max_streams;   /* B: independent streams decoded in lockstep (1 = the batch-1 path) */
    int32_t max_ctx;       /* positions per stream, at most the position table's rows */
    int32_t use_graph;     /* 1: replay captured HIP graphs of decode steps; 0: plain launches */
    int32_t head_grid;     /* blocks of the head's plate read (0: default) */
    int32_t graph_steps;   /* decode steps per captured graph, at most 16 (0: 16) */
    int32_t profile;       /* 1: launch the decode steps kernel by kernel (no graphs), each launch stamped with a HIP
                              event pair by its own dispatch (sm_profile, sm_profile_kernels) */
    int32_t table_mode;    /* the tables are read from memory; every loaded entry is compared with its defining
                              formula on the device at create.  1: refuse tables that differ (SM_E_IO); 0: accept
                              them (sm_info reports the check) */
    int32_t prefill_rows;  /* 0: the prompt runs position by position through the decode step; 1..64: every prompt
                              position but the last runs through the int8 MFMA banks that many rows a pass, each
                              weight read shared by the pass's rows (base2_stream.swift:74-91, 274-275: the
                              prompt through each layer at once); the last position is the first decode step */
    int32_t inv;           /* 1: the complement machine (base2_stream.swift:26 `inv`, "the whole machine on the
                              negative"): the stream row, every plate and every light held bit-complemented, each
                              pile corrected by the plate's column sum, the light's sum and the input count, stream
                              updates subtracted, the race won by the smallest complemented logit.  Its words, keys,
                              values and recorded intermediates are the plain machine's; SM_READ_RESID returns the
                              complemented stream.  GPT-2, max_streams 1, prefill_rows 0 */
    int32_t float_stages;  /* SM_FLOAT_* bits: those stages back in float64, as base2.py:10-11 switches them
                              (gauge=, edge=, arrival=; base2.py:66-69, 79-80, 89-92, 110-113) and
                              foundation0/pythia_base2.py:21-27 (gauge=, turn=, edge=, arrival=).  Diagnostics,
                              compared with the reference at the word level.  max_streams 1, prefill_rows 0, inv 0;
                              turn is the Pythia machine's (its layout's cosf.bin / sinf.bin).  With arrival the
                              cache holds each key as float64, not k16 / ek */
    int32_t top_read;      /* the head's read of the word table.  1: the collapsing top read (base2_stream_fr.swift:
                              4-15, its top=fr): the high-byte plane (w >> 8) for every word, each word's score
                              bounded exactly, the low bytes (w & 255) of the words that can still win; the same
                              words as the full read (GPT-2, max_streams 1, no inv or float stages, head_grid
                              393..512).  0: the full read (the default: measured faster at batch 1 since the
                              head's logits take a two-instruction rounding shift).  2: the collapsing read where
                              it applies, else the full read */
    int32_t att_split;     /* batch 1: decode steps at positions from this one on run the attention spread over the
                              GPU, each head's cached positions in chunks of 64, one block a chunk (the chunks'
                              scores and maxima, then arrivals against the head's maximum and the value sums added
                              exactly: two launches; the divisor and the output row are then formed by the next
                              phase's blocks); steps before it run one block a head.
                              0: from position 160; -1: never.  The same numbers either way (base2.py:85-100) */
    int32_t v64;           /* the value cache (base2.py's attention weighs each raw int64 value): every value's low
                              32 bits, and a row holding a value past 32 bits also whole; a head holding such a row
                              reads its values whole.  0: the others read the 32-bit rows alone (half the bytes);
                              1: every head reads its values whole from the start.  The same numbers either way.  Not
                              with the float arrival, whose cache holds int32 values (a value past 32 bits is
                              SM_E_OVERFLOW there) */
} sm_config;

enum { SM_FLOAT_GAUGE = 1, SM_FLOAT_EDGE = 2, SM_FLOAT_ARRIVAL = 4, SM_FLOAT_TURN = 8 };

/* Replaces base2_stream.swift:151-208 (device, pipelines, loading base2_gpu/ and its buffers) and
 * base2.py:12-16 (np.load of the converted model).  layout_dir is a base2_gpu.py directory
 * (base2_gpu.py:9-17: manifest.json, {bank}.wc/.e/.b, wte/wpe/phi/arrival/log2/exp2 .bin). */
int sm_create(const char* layout_dir, const sm_config* cfg, sm_machine** out);
int sm_destroy(sm_machine* m);

/* Empties every stream (positions, words, KV cache).  base2.py has no state; base2_stream.swift resets per
 * prompt at :264-271. */
int sm_reset(sm_machine* m);

/* Queues a prompt for one stream (base2_stream.swift:265-271: seq = ids, R0 rows from wte + wpe).  All
 * streams of one run must have prompts of the same length. */
int sm_prefill(sm_machine* m, int32_t stream, const int32_t* ids, int32_t n);

/* Runs the decode loop until every stream has n_words more greedy words; out is [n_streams][n_words].
 * Replaces base2.py:123 (got.append(forward(ids + got)) per word) and base2_stream.swift:273-281 (prompt,
 * then each word fed straight back on the device).  The first call also runs the prompt. */
int sm_generate(sm_machine* m, int32_t n_words, int32_t* out);

/* Records every intermediate of stream 0 at one position (-1: off).  Replaces fr2's rec=1 (recp kernel,
 * base2_stream_fr2.swift:564-570) and recording/C_plain.py's wrapped product. */
int sm_record_at(sm_machine* m, int32_t pos);

/* What sm_read returns (int64 unless noted). */
enum {
    SM_READ_K16 = 1,      /* int32 [768]  per-head 16-bit keys at (layer, stream, pos) */
    SM_READ_EK = 2,       /* int32 [12]   their water levels */
    SM_READ_V = 3,        /* int32 [768]  values (their low 32 bits; SM_READ_V64: whole) */
    SM_READ_RESID = 4,    /* [768] the stream R of `stream` after its last position */
    SM_READ_SEQ = 5,      /* int32 [max_ctx + 1] words per position of `stream` */
    SM_READ_REC_X16 = 10, /* [12][4][3072] light entering each bank (qkv, proj, fc, mproj) */
    SM_READ_REC_EXLS = 11,/* [12][4][2] its water level ex and gauge LS */
    SM_READ_REC_PILE = 12,/* [12][4][3072] piles */
    SM_READ_REC_QKV = 13, /* [12][2304] */
    SM_READ_REC_ATT = 14, /* [12][768] */
    SM_READ_REC_HID = 15, /* [12][3072] after the edge */
    SM_READ_REC_RESID = 16,/* [12][2][768] stream after each half layer */
    SM_READ_REC_HX16 = 17,/* [768] the head's light */
    SM_READ_REC_HEXLS = 18,/* [2] */
    SM_READ_REC_HPILE = 19,/* [vocab] */
    SM_READ_REC_LOGITS = 20,/* [vocab] gauged logits + standing amount (Pythia: plain logits, no bias) */
    /* the Pythia machine (foundation0/pythia_base2.py) only */
    SM_READ_REC_GAUGE = 21, /* [12][2][768] the gauge rows (ln1, ln2) of each layer (:100-110) */
    SM_READ_REC_FCPRE = 22, /* [12][3072] fc's plain output before the edge */
    SM_READ_REC_HGAUGE = 23,/* [768] the head's gauge row (lnf) */
    SM_READ_TOP = 24,       /* int64 [1 + 3 x 1024] the collapsing top read's last step: the survivor count, then
                               (word, exact pile, score) of the first 1024 survivors */
    SM_READ_V64 = 25        /* int64 [768]  the values at (layer, stream, pos), whole */
};
/* Copies one device array to host memory dst (bytes must match).  Replaces reading MTLBuffer contents
 * (base2_stream.swift:282-286) for per-intermediate parity. */
int sm_read(sm_machine* m, int32_t what, int32_t layer, int32_t stream, int32_t pos, void* dst, size_t bytes);

/* Head-launch timing gathered with profile = 1: launches seen and their summed duration (microseconds,
 * HIP events stamped by each head dispatch; with the collapsing top read, its first stage's).  clear = 1 empties the kernel-timing table afterwards.  Replaces fr2's
 * bench= timing (base2_stream_fr2.swift:1060-1075). */
int sm_profile(sm_machine* m, int64_t* n_heads, double* head_us, int32_t clear);

/* Kernel timing, process-wide.  Launches of a machine created with profile = 1 and, after sm_profile_stages(1),
 * of the stage and plate entry points are each stamped with a HIP event pair by their own dispatch (the interval a
 * kernel trace reports).  sm_profile_kernels waits for the device and returns, per kernel name, the launches and
 * their summed duration in microseconds since the last clear: names receives "name\tsymbol\n" a kernel (symbol: the
 * demangled device function with the most of those launches, as a kernel trace names it; names_bytes at most), launches and total_us at most max entries, *n how many; clear = 1 empties the table.
 * Replaces fr2's sbench= and pbench= timings of fused steps and plate reads (base2_stream_fr2.swift:1077-1149). */
int sm_profile_stages(int32_t on);
int sm_profile_kernels(char* names, int32_t names_bytes, int64_t* launches, double* total_us, int32_t max, int32_t* n,
                       int32_t clear);

/* Facts about a created machine: vocab, max_ctx, max_streams, rows of the position table, and whether every
 * loaded table entry equals its defining formula (base2_convert.py:48-61, checked on the device at create). */
/* Which machine a layout holds: 0 the GPT-2 machine of base2.py, 1 the Pythia machine of
 * foundation0/pythia_base2.py (a layout whose manifest says "kind": "pythia"); negative on error. */
int sm_model_kind(const sm_machine* m);
/* Which read of the word table the machine's decode steps use (base2_stream_fr.swift's top= switch, resolved
 * from sm_config.top_read): 1 the collapsing top read, 0 the full read; negative on error. */
int sm_top_read(const sm_machine* m);
int sm_info(const sm_machine* m, int32_t* vocab, int32_t* max_ctx, int32_t* max_streams, int32_t* n_pos,
            int32_t* tables_verified);

const char* sm_last_error(void);

/* ---------------------------------------------------------------------------------------------------
 * Stage entry points: base2.py's stage functions on caller-owned DEVICE buffers (unit parity, microbench).
 * stream is a hipStream_t (NULL: the null stream).  The tables come from sm_tables_create.
 * ------------------------------------------------------------------------------------------------- */
typedef struct sm_tables sm_tables;

/* the tables of base2_convert.py:48-61 (int64 host arrays, as in the npz) */
int sm_tables_create(const int64_t* phi, const int64_t* arrival, int32_t alen, const int64_t* log2t,
                     const int64_t* exp2t, int64_t log2_768, int64_t eps40, sm_tables** out);
int sm_tables_destroy(sm_tables* t);
/* 1 when every entry of the tables equals its defining formula (base2_convert.py:48-61), checked on the device at
 * sm_tables_create; 0 when one differs; negative on error */
int sm_tables_verified(const sm_tables* t);

int sm_stage_rshift(const int64_t* x, const int64_t* s, int64_t* out, int64_t n, void* stream);          /* base2.py:18-22 */
int sm_stage_log2fix(const sm_tables* t, const int64_t* v, int64_t* out, int64_t n, void* stream);       /* base2.py:42-48 */
int sm_stage_power(const sm_tables* t, const int64_t* x, const int64_t* F, int64_t* out, int64_t n, void* stream); /* base2.py:50-53 */
int sm_stage_edge(const sm_tables* t, const int64_t* h, int64_t* out, int64_t n, void* stream);          /* base2.py:78-83 */
int sm_stage_to16(const int64_t* X, int32_t rows, int32_t n, int64_t* x16, int64_t* ex, void* stream);  /* base2.py:24-27 */
int sm_stage_gauge_log(const sm_tables* t, const int64_t* R, int32_t rows, int64_t* x16, int64_t* ex,
                       int64_t* LS, void* stream);                                                      /* base2.py:55-60 */
int sm_stage_race(const int64_t* v, int64_t n, int64_t* out_index, void* stream);                       /* base2.py:34-40 */

/* One new position's attention for one stream (base2.py:85-100 for the last row; base2_stream.swift:120-133
 * without its 64-position cap).  qkv: device int64 [2304] (the gauged q, k, v of position pos); the caches,
 * head-major, hold positions < pos and receive position pos: k16 int16 [12][ctx][64] (the 16-bit keys, a
 * +32768 held as 32767), km int64 [12][ctx] (bit d set: dimension d of that key is +32768), ek int32 [12][ctx],
 * v int32 [12][ctx][64]; out: device int64 [768].  Zeroed caches are empty caches. */
int sm_stage_attend(const sm_tables* t, const int64_t* qkv, int16_t* k16, int64_t* km, int32_t* ek, int32_t* v,
                    int32_t pos, int32_t ctx, int64_t* out, void* stream);

/* The same attention as sm_stage_attend (the same arguments, caches and results), spread over the GPU as the batch-1
 * machine runs it from its att_split position on: each head's positions in chunks of 64, one block a chunk, three
 * launches (scores and chunk maxima; arrivals against the head's maximum with the value sums added exactly; the
 * divisor).  ctx at most 8192; the first call allocates its scratch (score row, chunk maxima, sums) with the tables. */
int sm_stage_attend_split(const sm_tables* t, const int64_t* qkv, int16_t* k16, int64_t* km, int32_t* ek, int32_t* v,
                          int32_t pos, int32_t ctx, int64_t* out, void* stream);

/* The same new position's attention for `rows` independent streams at once, through the batched machine's kernel
 * (one block per head and stream; base2.py:85-100 for each stream's last row).  qkv: device int64 [rows][2304]; the
 * caches are the same arrays per stream, stream-major: k16 int16 [rows][12][ctx][64], km int64 [rows][12][ctx],
 * ek int32 [rows][12][ctx], v int32 [rows][12][ctx][64]; out: device int64 [rows][768]. */
int sm_stage_attend_rows(const sm_tables* t, const int64_t* qkv, int32_t rows, int16_t* k16, int64_t* km, int32_t* ek,
                         int32_t* v, int32_t pos, int32_t ctx, int64_t* out, void* stream);

/* A plate on the device from an input-major int16 [nin][nout] host array: tile_cols > 0 lays it out for the
 * one-row GEMV (sm_plate_product), tile_cols == 0 as int8 MFMA byte planes for rows of lights
 * (sm_plate_product_rows, the batched streams' layout). */
typedef struct sm_plate sm_plate;
int sm_plate_create(const int16_t* w, const int32_t* e, const int64_t* b, int32_t nin, int32_t nout,
                    int32_t tile_cols, sm_plate** out);
int sm_plate_destroy(sm_plate* p);
/* pile[j] = sum_i x16[i] w[i][j], exact (base2.py:29-32; the split cells of base2_stream.swift:61-73).
 * x16: device int64 [nin] with values in [-32768, 32768]; pile: device int64 [nout]. */
int sm_plate_product(const sm_plate* p, const int64_t* x16, int64_t* pile, int32_t grid, void* stream);
/* pile[r][j] = sum_i x16[r][i] w[i][j] for rows r < rows <= 64, exact, through the int8 MFMA byte-plane
 * contraction (base2.py:29-32 for every row of a batch).  x16: device int64 [rows][nin] in [-32768, 32768];
 * pile: device int64 [rows][nout].  Calls on one plate share its light planes: serialise them. */
int sm_plate_product_rows(const sm_plate* p, const int64_t* x16, int32_t rows, int64_t* pile, void* stream);
/* The same product for a bank that forms its light from the producing phase's rows, as the batched machine's
 * proj and mproj do: pile[r][j] = sum_i to16(X[r])[i] w[i][j] (base2.py:24-27, then :29-32).  X: device int64
 * [rows][nin]; orw: device int64 [rows][12] (nin 768: one word per 64-value part, the attention's heads) or
 * [rows][192] (nin 3072: one per 16-value part, fc's column tiles), each the OR of |x| over its part (their OR is
 * the row's water level); pile: device int64 [rows][nout].  nout a multiple of 16 and at most 3072 (nin 768) or
 * a multiple of 48 (nin 3072); rows 1..64.  Calls on one plate share its scratch: serialise them. */
int sm_plate_product_rows_from(const sm_plate* p, const int64_t* X, const int64_t* orw, int32_t rows,
                               int64_t* pile, void* stream);
/* sm_plate_product_rows with no allocation on any call: the rows' light planes and row facts go to a static
 * device array of the library (590 KB, held by every GPU it runs on until the process ends), not to the plate's own
 * scratch.  No counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  rows 1..64 (more is refused with
 * SM_E_ARG); the same piles as sm_plate_product_rows.  Its launches are never timed (sm_profile_stages does not
 * apply: timing would create and record HIP events).  Every call on one GPU uses that GPU's one array, so calls
 * that overlap on one GPU (other streams, other threads) race; the caller serialises them. */
int sm_plate_product_rows_noalloc(const sm_plate* p, const int64_t* x16, int32_t rows, int64_t* pile, void* stream);
/* bytes of the device plate (for bandwidth accounting) */
int64_t sm_plate_bytes(const sm_plate* p);

#ifdef __cplusplus
}
#endif
#endif
