// Kernel argument blocks shared by the host code (sm_machine.hip) and the kernels (sm_kernels.hip).
#pragma once
#include "sm_device.h"

// prologue: how a phase forms its 16-bit light from the row it reads
enum { PRO_GAUGE = 0,   // gauge_log of the stream row R (768): x16, ex, LS (base2.py:55-60)
       PRO_TO16 = 1,    // to16 of an activation row (768 or 3072): x16, ex (base2.py:24-27)
       PRO_EMBED = 2,   // batched lights: the word enters, R = wte[word] + wpe[pos] (base2.py:103), then PRO_GAUGE
       PRO_X16 = 3,     // the light is given (int64 x16 values, ex = -16): the raw product test
       // batched streams: the producing bank's epilogue from its partial piles, then the light
       PRO_ADD_GAUGE = 4,   // R += rshift(pile, -(we + ex + 16)) + b, then PRO_GAUGE of R   (base2.py:105-106, 55-60)
       // the Pythia machine (foundation0/pythia_base2.py)
       PRO_PGAUGE = 6,      // its gauge with the norm's gain and offset, then to16 of that row     (:100-110, 113)
       // batch 1 with the attention spread over chunks of positions (sm_attend_split.hip): the row is the attention's
       // output, formed by every block from the heads' summed accumulators (aacc), then PRO_TO16 of it
       PRO_ATT = 7,         // GPT-2: power(num, -log2fix(Z))                                        (base2.py:99)
       PRO_PATT = 8,        // Pythia: the same power exact in 128 bits, with the reference's asserts (:139, 90)
       // batch 1 (GPT-2), layer 0's qkv: the race over the step before's head bests (base2.py:34-40, 114) and the
       // word fed back as the entering row wte[word] + wpe[q] (base2.py:103), in every block (block 0 writes the
       // word, the counters, the row and the next position), then PRO_GAUGE of that row: k_race1 folded in
       PRO_RACE = 9,
       // batched streams, layer 0's light: the race over the step before's head bests for the row's stream
       // (k_race_rows's arithmetic; block 0 writes the counters and the next position slot), then PRO_EMBED of the
       // word it feeds back
       PRO_RACE_EMBED = 10 };
// epilogue: what a phase does with each finished pile
enum { EPI_GAUGED = 0,       // power(pile, (we + ex + 16) 65536 - LS) + b          (base2.py:70-71)
       EPI_GAUGED_EDGE = 1,  // the same, then the edge                               (base2.py:106, 78-83)
       EPI_PLAIN_ADD = 2,    // R += rshift(pile, -(we + ex + 16)) + b                  (base2.py:73-76, 105-106)
       EPI_HEAD = 3,         // gauged logit + standing amount, then the race           (base2.py:107-114)
       EPI_PILE = 4,         // the raw pile (product only)                             (base2.py:29-32)
       EPI_PART = 5,         // batched: the int32 accumulators, finished by the consumer's prologue
       // the Pythia machine: every plate is plain (foundation0/pythia_base2.py:112-114)
       EPI_PLAIN = 6,        // rshift(pile, -(we + ex + 16)) + b, written
       EPI_PLAIN_EDGE = 7,   // the same, then the edge (:147)
       EPI_PHEAD = 8,        // rshift(pile, -(we + ex + 16)) with no bias, then the race (:158-160)
       // the collapsing top read (base2_stream_fr.swift:4-15): the high-byte plane's coarse pile and each word's
       // exact bounds, the block's best low and its candidates
       EPI_TOP1 = 9,
       // batched Pythia: R += rshift(pile, -(we + ex + 16)) + b and the other half's plain bank, finished here from
       // its K-slice partial piles (the parallel residual, foundation0/pythia_base2.py:155-157)
       EPI_PLAIN_ADD2 = 10 };

// k_gemv's MODE bits (batch 1): the complement machine, two of the stages back in float64 (base2.py:10-11,
// foundation0/pythia_base2.py:21-27: diagnostics that put one stage back to float; compared at the word level), and
// plates of 17-bit digits
enum { MODE_INV = 1,       // the complement machine (see race_beats)
       MODE_FGAUGE = 2,    // gauge=float: GPT-2 base2.py:66-69, 110-113; Pythia foundation0/pythia_base2.py:102-104
       MODE_FEDGE = 4,     // edge=float: GPT-2's tanh form base2.py:79-80; Pythia's erf form pythia_base2.py:144-146
       MODE_SPLIT = 8 };   // every digit held as the difference of two int16 digits, w = W - W2 (the Pythia machine's
                           // plates=built, foundation0/pythia_base2.py:44-46: finished - start, 17 bits a digit); the
                           // pile is the exact integer sum x . W - x . W2

// Record of one position's intermediates (stream 0), written when the position equals *pos.
struct Rec {
    const int* pos;
    i64* x16;    // [L][4][3072]
    i64* exls;   // [L][4][2]
    i64* pile;   // [L][4][3072]
    i64* qkv;    // [L][2304]
    i64* att;    // [L][768]
    i64* hid;    // [L][3072]
    i64* resid;  // [L][2][768]
    i64* hx16;   // [768]
    i64* hexls;  // [2]
    i64* hpile;  // [vocab]
    i64* logits; // [vocab]
};

// batch 1's race over the head blocks' bests and the next entering row (k_race1, k_embed1, PRO_RACE)
struct Race1Args {
    const i64* part_v; const int* part_i; int nblk;
    int* seq; int* words; int* pos; const int* plen; int* nwords;
    int* pos_next;              // PRO_RACE: the position slot the race writes (pos holds the step before's)
    i64* R0;                    // the entering row of the next position
    int npos;                   // rows of the position table (GPT-2): no entering row past it
    const i64* wte; const i64* wpe;             // GPT-2
    const short* ew; const int* ee;             // Pythia
    const short* ew2;                           // Pythia, split word table (plates=built): the row is ew - ew2
};

struct GemvArgs {
    const int4* W;              // the plate in column tiles of TC (see sm_machine.hip: tile_plate)
    const int4* W2;             // MODE_SPLIT: the subtracted plate, tiled as W
    const int* we;              // per-column power of two
    const i64* bias;            // per-column bias (2^-16)
    const i64* sw;              // MODE_INV: each column's sum over the plain plate (W holds ~w)
    int nout, ntiles;
    const i64* X;               // the row this phase reads (PRO_GAUGE / PRO_TO16 / PRO_X16 / PRO_PGAUGE)
    i64* Y;                     // output row (or the stream R for EPI_PLAIN_ADD)
    const i64* Yb;              // EPI_PLAIN_ADD: the row added to (null: Y itself; layer 0: the entering row)
    Tables tb;
    // record slot for this phase (layer l, bank k) or null; read only by the REC = 1 instantiations
    i64* rx16; i64* rexls; i64* rpile; i64* rout;
    const int* pos;             // device position counter
    const int* rec_pos;         // record when the position equals *rec_pos
    // head only: each block's best word
    i64* part_v; int* part_i;
    i64* rlogits;
    // the Pythia machine: the norm this phase's gauge uses, extra record slots
    const int* ng; const i64* nb; int nge;     // gain (16 places), offset (2^-16), the gain's power of two
    i64* rg;                                   // record: the gauge's output row
    i64* rout2;                                // record: EPI_PLAIN_EDGE's row after the edge (rout: before)
    // EPI_TOP1: each block's candidates (word, high bound, coarse pile) in slots [block][TOP_CAP], their count in
    // part_i[block] and the block's best low in part_v[block]; block 0 also writes the light (tx: 768 values) and
    // its facts (tf: ex, LS, EXP2 of the fine part)
    int* cand_j; i64* cand_h; i64* cand_c;
    int* tx; i64* tf;
    // the next GEMV phase's plate, requested while this phase runs: block b requests the 128-byte lines that the
    // next kernel's blocks b, b + gridDim.x, .. read first.  The lines pass through the memory-side Infinity Cache,
    // which then serves the next phase's first requests (its own L2 misses them: measured by FETCH_SIZE); null: none
    int* err;                                  // the Pythia machine: its rshift assert sets SM_ERR_RANGE here
    const char* pf; int pf_lines; int pf_nblk;       // plate, lines a next-kernel block reads, the next grid
    int pf_total;                                    // the plate's lines (none past them is requested)
    // PRO_ATT / PRO_PATT: the heads' accumulators [12][68] (64 value sums, the arrival sum, the largest weighed |v|)
    // and the attention row's record slot (block 0 writes it at the recorded position)
    const i64* aacc; i64* ratt;
    // PRO_RACE: the race of the step before (its head's bests, the word fed back, the counters, the entering row)
    Race1Args race;
};
#define TOP_ITERS 8                 // EPI_TOP1: tiles a wave may finish (the grid is sized for it)

// The complement machine (base2_stream.swift:26 `inv`, "the whole machine on the negative"): the stream row, every
// plate and every light are held bit-complemented (~x = -x - 1).  A pile is then
//   sum (~w)(~x) = sum w x + sum w + sum x + nin,
// so the plain pile is the product less the plate's column sum, the light's sum and the input count
// (:72, :90); a stream update ~R - a = ~(R + a) subtracts (:108); the race reads the complemented logits and the
// smallest wins, ties to the lowest word (:134-139); the entering row is ~(wte + wpe) (:146, :271).
// "a beats b" for a race entry (value, word); word < 0: no entry
template <int INV>
SMD bool race_beats(i64 a, int ai, i64 b, int bi) {
    return ai >= 0 && (bi < 0 || (INV ? a < b : a > b) || (a == b && ai < bi));
}

// Batch 1: the race over the head blocks' bests, the word fed back, and the next position's entering row
// (base2.py:103: wte[word] + wpe[p]; foundation0/pythia_base2.py:153: rshift(embed.w[word], -(embed.e[word] + 16)))


// The collapsing top read's second stage, batch 1 (one block): the survivors' low bytes, their exact scores, the
// race, then k_race1's word feed and entering row
struct TopArgs {
    Race1Args r;                    // part_v: the first stage's block lows; part_i: their candidate counts
    int cap;                        // candidate slots a block
    const int* cand_j; const i64* cand_h; const i64* cand_c;
    const int* tx; const i64* tf;   // the light and its facts (from the first stage's block 0)
    const unsigned char* lo;        // [vocab][768] each word's low bytes (w & 255), word by word
    const int* we; const i64* bias;
    Tables tb;
    int* tn; int* tw; i64* tpile; i64* tscore; int tmax;   // the step's survivors: count, word, exact pile, score
};

struct AttArgs {
    const i64* QKV;     // [B][2304]
    // the cache, head-major so that a (stream, head)'s positions are contiguous: [B][12 heads][ctx][64]
    short* K16;         // [B][12][ctx][64] per-head 16-bit keys (values in [-32768, 32768]; +32768 held as 32767)
    i64* KM;            // [B][12][ctx]     bit d: dimension d of the key is +32768 (one more than K16 holds)
    int* EK;            // [B][12][ctx]     their water levels
    int* V;             // [B][12][ctx][64] raw gauged values: their low 32 bits (every value that fits 32 bits)
    i64* V64;           // [B][12][ctx][64] (when non-null) a row holding a value past 32 bits, whole (base2.py
                        // keeps int64 values); rows that fit 32 bits are not written here
    int* VW;            // [B][12][ctx] (with V64) nonzero: row p is in V64 (one of its values is past 32 bits)
    int* vbig;          // [B][12] (with V64) nonzero: the (stream, head) holds a value past 32 bits, and the
                        // attention reads that head's values whole (V64 where VW marks the row, else V)
    i64* out;           // [B][768]
    int* out32;         // [B][768] (when non-null): the same values' low 32 bits, for a consumer that reads a
                        // row's 32-bit copy wherever its OR words show that the row fits (k_gemm's SRC path)
    i64* out_or;        // [B][12] (when non-null): OR of |out| over each head's 64 values, the next light's
                        // water level without a pass over the row
    const int* pos;     // position being written and read up to (inclusive)
    int ctx;
    Tables tb;
    int* err;           // bit 0: a value left 32 bits with no V64 to hold it; bit 1: a value the reference asserts on
    const int* rec_pos; i64* ratt;
    // the Pythia machine: turns on the first rot dims of q and k, the scores' half-log2(head size)
    const int* cosT; const int* sinT;   // [npos][rot / 2] at 2^-30
    const double* cosF; const double* sinF;   // turn=float: [npos][rot / 2] float64 (pythia_base2.py:118-119)
    double* KF;         // arrival=float: [12][ctx][64] each cached key as float64 (its raw gauged value)
    int rot; i64 half; i64 ehalf;       // ehalf = EXP2[(-half) & 0xFFFF]
    // prompt rows: row r is position rowmap[r] & 0xFFFF of stream rowmap[r] >> 16 (null: row r is stream r at
    // *pos).  Their keys and values are in the cache already (k_kv_rows), so the attention only reads it.
    const int* rowmap;
    // the batch-1 attention spread over chunks of positions (k_att_scores, k_att_mix, k_att_finish): the score row
    // [12][ctx], the chunk maxima [12][ncm], the per-head accumulators [12][ACC_W]
    i64* asc; i64* acm; i64* aacc; int ncm;
};

// error bits in the device error word
#define SM_ERR_V32 1
#define SM_ERR_RANGE 2
