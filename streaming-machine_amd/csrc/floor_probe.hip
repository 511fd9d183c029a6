// The decode step's launch-structure floor, measured.  Batch 1: the step's dependent launches (12 layers x
// [qkv, attend, proj, fc, mproj], the head) with the machine's grids and block sizes, replayed from a HIP graph of
// 15 steps as the machine runs them: a step after the first takes the race of the step before into its layer-0
// qkv (every block reads the head's 512 bests and the chosen word's row), and the race runs once, after the last
// step (61 launches a step, 916 a graph); two forms:
//   empty  - every kernel returns at once: the cost of the dependent launches alone;
//   bytes  - every kernel reads the row it depends on (the previous kernel's output) and its share of its plate
//            (the GPT-2 124M shapes: int16 plates of 768x2304, 768x768, 768x3072, 3072x768, and the 768 x 50257
//            word table, read whole as the machine's default head does), the attention reads 16 cached positions
//            of keys (int16) and values
//            (int32) per head, and each kernel writes its outputs -- no arithmetic beyond folding what it read.
// The machine's step does all of this plus its arithmetic, so its time over "bytes" is what the arithmetic,
// the block reductions and the table reads cost.
// 64 streams ("b64"): the batched step's 86 launches (the word's light with the race of the step before, a row a
// block, stood in for by the race kernel; 12 layers x [qkv, attend, proj, light, fc, mproj partials, light]; the
// head) with the machine's grids, graphs of 16 steps, the same two forms; in
// "bytes" each bank block reads its row tile's light planes or int32 rows and its plate share, each attention
// block 96 positions of its cache rows (38 KB), each light block its row (and the partials), the head its plate.
// The Pythia machine at 32 streams ("pythia32"): its 50 launches a step (the words entering with the race of the
// step before, 12 x [fc | qkv, the attention | mproj partials, proj, the row kernel], the head; the race once after
// a graph's last step) with the machine's grids, graphs of 16 steps,
// the same two forms; the attention blocks read 192 positions of cache rows (the workload's mean context).
// Prints one JSON line with both.  With the argument "persist": batch 1 as one persistent kernel (below), its step
// time and, on stderr, block 0's hand-off times in the last step.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <string>

#define CHK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { fprintf(stderr, "floor_probe: %s at line %d\n", hipGetErrorString(e_), __LINE__); return 1; } } while (0)
typedef long long i64;
typedef int v4i __attribute__((ext_vector_type(4)));

// a GEMV-shaped phase: NIN-wide row, tiles of TC columns (WB bytes a weight), WPB waves a block, each wave its
// tiles t, t + grid waves, ..; HEADK: one output a block (the head's block best) instead of one a column
template <int NIN, int TC, int WPB, int WB, bool EMPTY, bool HEADK = false>
__global__ __launch_bounds__(64 * WPB) void k_floor_phase(const i64* X, const v4i* W, int ntiles, i64* Y) {
    if (EMPTY) return;
    constexpr int NT = 64 * WPB, PER = NIN / NT, U = TC * NIN * WB / 16 / 64;
    static_assert(NIN % NT == 0 && TC * NIN * WB % (16 * 64) == 0, "the row and the tile split evenly");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    i64 acc = 0;
#pragma unroll
    for (int m = 0; m < PER; m++) acc ^= X[tid + NT * m];
    i64 best = 0;
    for (int t = blockIdx.x * WPB + wave; t < ntiles; t += gridDim.x * WPB) {
        const v4i* base = W + (size_t)t * (TC * NIN * WB / 16) + lane;
        i64 a = acc;
#pragma unroll
        for (int m = 0; m < U; m++) { const v4i w = base[64 * m]; a += w.x ^ w.y ^ w.z ^ w.w; }
        a += __shfl_xor(a, 1, 64);
        if (HEADK) best = a > best ? a : best;
        else if (lane < TC) Y[t * TC + lane] = a;
    }
    if (HEADK && tid == 0) Y[blockIdx.x] = best;
}
// layer 0's qkv with the race of the step before: the head's 512 bests (two a thread), their maximum over the
// block, the chosen word's row as the entering row (block 0 writes it), then the qkv phase's tiles
template <bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_qkv_race(const i64* part, const i64* wte, int nwords, const v4i* W,
                                                        int ntiles, i64* Y, i64* R0) {
    if (EMPTY) return;
    __shared__ i64 wb[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    i64 b = max(part[tid], part[tid + 256]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, __shfl_xor(b, o, 64));
    if (lane == 0) wb[wave] = b;
    __syncthreads();
    b = max(max(wb[0], wb[1]), max(wb[2], wb[3]));
    const int word = (int)((unsigned long long)b % (unsigned)nwords);
    i64 acc = 0;
#pragma unroll
    for (int m = 0; m < 3; m++) {
        const i64 x = wte[(size_t)word * 768 + tid + 256 * m];
        acc ^= x;
        if (blockIdx.x == 0) R0[tid + 256 * m] = x;
    }
    for (int t = blockIdx.x * 4 + wave; t < ntiles; t += gridDim.x * 4) {
        const v4i* base = W + (size_t)t * (2 * 768 * 2 / 16) + lane;
        i64 a = acc;
#pragma unroll
        for (int m = 0; m < 3; m++) { const v4i w = base[64 * m]; a += w.x ^ w.y ^ w.z ^ w.w; }
        a += __shfl_xor(a, 1, 64);
        if (lane < 2) Y[t * 2 + lane] = a;
    }
}
// one wave a head: the new q, k, v and P cached positions of the head's keys and values
template <bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_attend(const i64* QKV, const short* K, const int* V, int P, int ctx, i64* out) {
    if (EMPTY || threadIdx.x >= 64) return;
    const int h = blockIdx.x, lane = threadIdx.x;
    i64 s = QKV[h * 64 + lane] ^ QKV[768 + h * 64 + lane] ^ QKV[1536 + h * 64 + lane];
    const short* Kh = K + (size_t)h * ctx * 64;
    const int* Vh = V + (size_t)h * ctx * 64;
    for (int r = 0; r < P; r++) s += Kh[r * 64 + lane] + Vh[r * 64 + lane];
    out[h * 64 + lane] = s;
}
// one block: the head blocks' bests, then the chosen word's row of the word table written as the next entering row
template <bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_race(const i64* part, int n, const i64* wte, int nwords, i64* R0) {
    if (EMPTY) return;
    i64 b = 0;
    for (int i = threadIdx.x; i < n; i += 256) b = part[i] > b ? part[i] : b;
    b = max(b, __shfl_xor(b, 1, 64));
    const int word = (int)((unsigned long long)b % (unsigned)nwords);
    for (int i = threadIdx.x; i < 768; i += 256) R0[i] = wte[(size_t)word * 768 + i] + b;
}

template <bool EMPTY>
static int run(double& us) {
    const size_t qkvB = 768 * 2304 * 2, projB = 768 * 768 * 2, fcB = 768 * 3072 * 2, mpB = 3072 * 768 * 2;
    const int head_tiles = (50257 + 3) / 4;                     // 4-column tiles of the int16 word table
    const size_t headB = (size_t)head_tiles * 4 * 768 * 2, layerB = qkvB + projB + fcB + mpB;
    const int CTX = 64, P = 16, WTE = 1024, STEPS = 15, REPS = 20;
    char* plates = nullptr;
    i64 *R, *QKV, *att, *hid, *part, *wte;
    short* K;
    int* V;
    CHK(hipMalloc(&plates, 12 * layerB + headB));
    CHK(hipMalloc(&R, 768 * 8)); CHK(hipMalloc(&QKV, 2304 * 8)); CHK(hipMalloc(&att, 768 * 8)); CHK(hipMalloc(&hid, 3072 * 8));
    CHK(hipMalloc(&part, 512 * 8)); CHK(hipMalloc(&wte, (size_t)WTE * 768 * 8));
    CHK(hipMalloc(&K, (size_t)12 * 12 * CTX * 64 * 2)); CHK(hipMalloc(&V, (size_t)12 * 12 * CTX * 64 * 4));
    CHK(hipMemset(plates, 1, 12 * layerB + headB));
    CHK(hipMemset(R, 0, 768 * 8)); CHK(hipMemset(QKV, 0, 2304 * 8)); CHK(hipMemset(att, 0, 768 * 8));
    CHK(hipMemset(hid, 0, 3072 * 8)); CHK(hipMemset(part, 0, 512 * 8)); CHK(hipMemset(wte, 0, (size_t)WTE * 768 * 8));
    CHK(hipMemset(K, 0, (size_t)12 * 12 * CTX * 64 * 2)); CHK(hipMemset(V, 0, (size_t)12 * 12 * CTX * 64 * 4));
    CHK(hipDeviceSynchronize());
    hipStream_t st;
    CHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int s = 0; s < STEPS; s++) {
        const char* pl = plates;
        for (int l = 0; l < 12; l++) {
            const v4i* wq = (const v4i*)pl; pl += qkvB;
            const v4i* wp = (const v4i*)pl; pl += projB;
            const v4i* wf = (const v4i*)pl; pl += fcB;
            const v4i* wm = (const v4i*)pl; pl += mpB;
            const size_t kv = (size_t)l * 12 * CTX * 64;
            if (l == 0 && s > 0) k_floor_qkv_race<EMPTY><<<288, 256, 0, st>>>(part, wte, WTE, wq, 1152, QKV, R);
            else k_floor_phase<768, 2, 4, 2, EMPTY><<<288, 256, 0, st>>>(R, wq, 1152, QKV);
            k_floor_attend<EMPTY><<<12, 256, 0, st>>>(QKV, K + kv, V + kv, P, CTX, att);
            k_floor_phase<768, 2, 2, 2, EMPTY><<<192, 128, 0, st>>>(att, wp, 384, R);
            k_floor_phase<768, 2, 4, 2, EMPTY><<<384, 256, 0, st>>>(R, wf, 1536, hid);
            k_floor_phase<3072, 1, 4, 2, EMPTY><<<192, 256, 0, st>>>(hid, wm, 768, R);
        }
        k_floor_phase<768, 4, 4, 2, EMPTY, true><<<512, 256, 0, st>>>(R, (const v4i*)pl, head_tiles, part);
        if (s == STEPS - 1) k_floor_race<EMPTY><<<1, 256, 0, st>>>(part, 512, wte, WTE, R);
    }
    CHK(hipStreamEndCapture(st, &g));
    CHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0)); CHK(hipEventCreate(&e1));
    for (int i = 0; i < 3; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipStreamSynchronize(st));
    CHK(hipEventRecord(e0, st));
    for (int i = 0; i < REPS; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipEventRecord(e1, st));
    CHK(hipStreamSynchronize(st));
    float ms = 0.0f;
    CHK(hipEventElapsedTime(&ms, e0, e1));
    us = ms * 1000.0 / (REPS * STEPS);
    CHK(hipEventDestroy(e0)); CHK(hipEventDestroy(e1));
    CHK(hipGraphExecDestroy(ge)); CHK(hipGraphDestroy(g)); CHK(hipStreamDestroy(st));
    for (void* q : {(void*)plates, (void*)R, (void*)QKV, (void*)att, (void*)hid, (void*)part, (void*)wte, (void*)K, (void*)V})
        CHK(hipFree(q));
    return 0;
}

// ---- 64 streams ----
// a block reads NA int4 a thread of A (region blockIdx.y ra + blockIdx.x rax) and NB of B (region blockIdx.x rb),
// then writes NOUT values
template <int NT, int NA, int NB, int NOUT, bool EMPTY, int ID>
__global__ __launch_bounds__(NT) void k_floor_move(const v4i* A, size_t ra, size_t rax, const v4i* B, size_t rb, i64* out) {
    if (EMPTY) return;
    const int tid = threadIdx.x;
    const v4i* a = A + (size_t)blockIdx.y * ra + (size_t)blockIdx.x * rax + tid;
    const v4i* b = B + (size_t)blockIdx.x * rb + tid;
    int s = 0;
#pragma unroll
    for (int i = 0; i < NA; i++) { const v4i v = a[(size_t)NT * i]; s += v.x ^ v.y ^ v.z ^ v.w; }
#pragma unroll
    for (int i = 0; i < NB; i++) { const v4i v = b[(size_t)NT * i]; s += v.x ^ v.y ^ v.z ^ v.w; }
    const size_t blk = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    for (int i = tid; i < NOUT; i += NT) out[blk * NOUT + i] = s + i;
}
// the head: each block its waves' light planes (NP v4 a thread: 24 for four row tiles), then its share of the plate
template <bool EMPTY, int NP = 24>
__global__ __launch_bounds__(256) void k_floor_head64(const v4i* planes, const v4i* W, size_t nW, i64* part) {
    if (EMPTY) return;
    const int tid = threadIdx.x;
    int s = 0;
#pragma unroll
    for (int i = 0; i < NP; i++) { const v4i v = planes[tid + 256 * i]; s += v.x ^ v.y; }
    for (size_t i = (size_t)blockIdx.x * 256 + tid; i < nW; i += (size_t)gridDim.x * 256) { const v4i v = W[i]; s += v.x ^ v.w; }
    if (tid < 64) part[(size_t)blockIdx.x * 64 + tid] = s;
}
template <bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_race64(const i64* part, i64* R) {
    if (EMPTY) return;
    i64 b = 0;
    for (int i = threadIdx.x; i < 512; i += 256) b = max(b, part[(size_t)i * 64 + blockIdx.x]);
    b = max(b, __shfl_xor(b, 1, 64));
    if (threadIdx.x == 0) R[blockIdx.x] = b;
}

template <bool EMPTY>
static int run64(double& us) {
    const size_t qkvB = 768 * 2304 * 2, projB = 768 * 768 * 2, fcB = 768 * 3072 * 2, mpB = 3072 * 768 * 2;
    const size_t headB = (size_t)768 * 50272 * 2, layerB = qkvB + projB + fcB + mpB;
    const size_t kvL = (size_t)64 * 12 * 160 * 396;          // a layer's cache: 64 streams x 12 heads x 160 positions
    const size_t planesB = 4 * 36864 * 2, rowsB = (size_t)64 * 3072 * 8, partsB = (size_t)4 * 3 * 64 * 768 * 4, NOUTV = 1 << 19;
    const int STEPS = 16, REPS = 10;
    char *plates = nullptr, *planes, *rows, *parts, *kv;
    i64* out;
    CHK(hipMalloc(&plates, 12 * layerB + headB)); CHK(hipMalloc(&planes, planesB)); CHK(hipMalloc(&rows, rowsB));
    CHK(hipMalloc(&parts, partsB)); CHK(hipMalloc(&kv, 12 * kvL)); CHK(hipMalloc(&out, NOUTV * 8));
    CHK(hipMemset(plates, 1, 12 * layerB + headB)); CHK(hipMemset(planes, 1, planesB)); CHK(hipMemset(rows, 1, rowsB));
    CHK(hipMemset(parts, 1, partsB)); CHK(hipMemset(kv, 1, 12 * kvL)); CHK(hipMemset(out, 0, NOUTV * 8));
    CHK(hipDeviceSynchronize());
    hipStream_t st;
    CHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    const v4i *P = (const v4i*)planes, *Rw = (const v4i*)rows, *Pa = (const v4i*)parts;
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int s = 0; s < STEPS; s++) {
        const char* pl = plates;
        for (int l = 0; l < 12; l++) {
            const v4i* wq = (const v4i*)pl; pl += qkvB;
            const v4i* wp = (const v4i*)pl; pl += projB;
            const v4i* wf = (const v4i*)pl; pl += fcB;
            const v4i* wm = (const v4i*)pl; pl += mpB;
            const v4i* kvl = (const v4i*)(kv + l * kvL);
            // qkv: the row tile's light planes (36 KB) and the column tile's plate (24 KB)
            k_floor_move<256, 9, 6, 256, EMPTY, 1><<<dim3(144, 4), 256, 0, st>>>(P, 2304, 0, wq, 1536, out);
            // attention: each (head, stream) block 96 positions of its cache rows (38 KB)
            k_floor_move<256, 9, 0, 64, EMPTY, 2><<<dim3(12, 64), 256, 0, st>>>(kvl, 12 * 2376, 2376, kvl, 0, out);
            // proj: the tile's attention rows at 32 bits (48 KB) and its plate (24 KB)
            k_floor_move<256, 12, 6, 256, EMPTY, 3><<<dim3(48, 4), 256, 0, st>>>(Rw, 3072, 0, wp, 1536, out);
            // the stream's light: a row (6 KB) a block
            k_floor_move<192, 2, 0, 288, EMPTY, 4><<<dim3(1, 64), 192, 0, st>>>(Rw, 384, 0, Rw, 0, out);
            // fc: light planes (36 KB) and plate (24 KB)
            k_floor_move<256, 9, 6, 256, EMPTY, 5><<<dim3(192, 4), 256, 0, st>>>(P, 2304, 0, wf, 1536, out);
            // mproj partials: the tile's hidden rows of its K slice at 32 bits (48 KB) and three column tiles (72 KB)
            k_floor_move<256, 12, 18, 1152, EMPTY, 6><<<dim3(64, 4), 256, 0, st>>>(Rw, 3072, 0, wm, 4608, out);
            // mproj's finish and the next light: four slices' partials (36 KB) and the row a block
            k_floor_move<192, 12, 2, 1056, EMPTY, 7><<<dim3(1, 64), 192, 0, st>>>(Pa, 2304, 0, Rw, 0, out);
        }
        k_floor_head64<EMPTY><<<512, 256, 0, st>>>(P, (const v4i*)pl, headB / 16, out);
        k_floor_race64<EMPTY><<<64, 256, 0, st>>>(out, out + (1 << 18));
    }
    CHK(hipStreamEndCapture(st, &g));
    CHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0)); CHK(hipEventCreate(&e1));
    for (int i = 0; i < 2; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipStreamSynchronize(st));
    CHK(hipEventRecord(e0, st));
    for (int i = 0; i < REPS; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipEventRecord(e1, st));
    CHK(hipStreamSynchronize(st));
    float ms = 0.0f;
    CHK(hipEventElapsedTime(&ms, e0, e1));
    us = ms * 1000.0 / (REPS * STEPS);
    CHK(hipEventDestroy(e0)); CHK(hipEventDestroy(e1));
    CHK(hipGraphExecDestroy(ge)); CHK(hipGraphDestroy(g)); CHK(hipStreamDestroy(st));
    for (void* q : {(void*)plates, (void*)planes, (void*)rows, (void*)parts, (void*)kv, (void*)out}) CHK(hipFree(q));
    return 0;
}

// ---- batch 1 as one persistent kernel ----
// The same step's phases inside one cooperative launch of 256 blocks (one a CU, co-resident by the launch's
// guarantee), each phase's outputs handed to the next through memory with no kernel boundary.  A row entry is two
// 64-bit words, each a 32-bit tag (the phase's sequence number, never 0) and one half of the value, written and read
// with agent-scope relaxed 64-bit atomics: a reader takes an entry once both of its words carry the sequence number
// it waits for, so the data arrives with its own flag (no fence, no separate flag word, no second read).  Every block
// requests its share of the next phase's plate before it waits for the row it needs.  Every wait is bounded by the
// constant clock: past the limit the block sets the error word and leaves the kernel, and so does every block
// waiting on it, so the launch always ends.
// Per step: 12 layers x [qkv (2304 outputs, 9 a block), attention (blocks 0-11, a head each, reading only their
// head's q, k, v entries and 16 cached positions), proj (768, 3 a block), fc (3072, 12 a block), mproj (768)], the
// head (each block 1/256 of the word table, its best), then the race in every block (the 256 bests) and the next
// entering row read from the word table by every block: 61 hand-offs a step.
#define PP_NB 256
#define PP_ROW 3072                      // entries a row slot holds
#define PP_SLOTS 62
struct PersistArgs {
    const v4i* plates;                   // 12 layers (qkv, proj, fc, mproj) then the head's table, as in run()
    unsigned long long* rows;            // [PP_SLOTS][PP_ROW][2] tagged entries
    const short* K; const int* V;        // the cache, as in run()
    const i64* wte;
    int* err;                            // 1: a wait passed its limit
    i64* sink;
    long long* stamps;                   // block 0, the last step: the constant clock after each hand-off
    int steps, ctx, P;
    long long limit;                     // constant-clock ticks (100 MHz) a wait may take
};
__device__ __forceinline__ void pp_put(unsigned long long* rows, int slot, int i, unsigned tag, i64 v) {
    unsigned long long* e = rows + ((size_t)slot * PP_ROW + i) * 2;
    __hip_atomic_store(e, ((unsigned long long)tag << 32) | (unsigned)(unsigned long long)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(e + 1, ((unsigned long long)tag << 32) | (unsigned)((unsigned long long)v >> 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// entries [i0, i0 + n) of a slot into LDS x[] once every one carries tag; false (the block leaves) past the limit.
// A thread's entries (at most E) are requested together each round, so a round is one memory round trip.
template <int E>
__device__ bool pp_get(const PersistArgs& a, int slot, int i0, int n, unsigned tag, i64* x, long long t0, int sidx = -1) {
    const unsigned long long* base = a.rows + ((size_t)slot * PP_ROW + i0) * 2;
    unsigned want = 0;
#pragma unroll
    for (int k = 0; k < E; k++)
        if ((int)threadIdx.x + 256 * k < n) want |= 1u << k;
    bool late = false;
    while (want) {
        unsigned long long lo[E], hi[E];
#pragma unroll
        for (int k = 0; k < E; k++) {
            const int i = (want >> k) & 1 ? (int)threadIdx.x + 256 * k : 0;
            lo[k] = __hip_atomic_load(base + 2 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            hi[k] = __hip_atomic_load(base + 2 * i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int k = 0; k < E; k++) {
            if (((want >> k) & 1) && (unsigned)(lo[k] >> 32) == tag && (unsigned)(hi[k] >> 32) == tag) {
                x[threadIdx.x + 256 * k] = (i64)(((hi[k] & 0xFFFFFFFFull) << 32) | (lo[k] & 0xFFFFFFFFull));
                want &= ~(1u << k);
            }
        }
        if (want && (long long)__builtin_amdgcn_s_memrealtime() - t0 > a.limit) { late = true; break; }
    }
    if (__syncthreads_or(late)) {
        if (threadIdx.x == 0) atomicOr(a.err, 1);
        return false;
    }
    if (sidx >= 0 && blockIdx.x == 0 && threadIdx.x == 0) a.stamps[sidx] = (long long)__builtin_amdgcn_s_memrealtime();
    return true;
}
// a phase's share of a plate: bytes [b * share, (b + 1) * share) of it, PL v4 a thread at most (clamped to the plate)
template <int PL>
__device__ __forceinline__ void pp_fetch(v4i (&w)[PL], const v4i* plate, size_t n16) {
    const size_t share = (n16 + PP_NB - 1) / PP_NB, b0 = (size_t)blockIdx.x * share;
#pragma unroll
    for (int m = 0; m < PL; m++) {
        size_t i = b0 + threadIdx.x + (size_t)blockDim.x * m;
        const bool in = i < b0 + share && i < n16;
        w[m] = plate[in ? i : 0];
        if (!in) w[m] = v4i{0, 0, 0, 0};
    }
}
template <int PL>
__device__ __forceinline__ i64 pp_fold(const v4i (&w)[PL]) {
    i64 s = 0;
#pragma unroll
    for (int m = 0; m < PL; m++) s += w[m].x ^ w[m].y ^ w[m].z ^ w[m].w;
    return s;
}
__device__ __forceinline__ i64 pp_rowsum(const i64* x, int n, i64* red) {
    i64 s = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s ^= x[i];
    for (int o = 32; o > 0; o >>= 1) s ^= __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = red[0] ^ red[1] ^ red[2] ^ red[3];
    __syncthreads();
    return s;
}
__global__ __launch_bounds__(256) void k_persist(PersistArgs a) {
    constexpr size_t qkvB = 768 * 2304 * 2, projB = 768 * 768 * 2, fcB = 768 * 3072 * 2, mpB = 3072 * 768 * 2;
    constexpr size_t layer16 = (qkvB + projB + fcB + mpB) / 16, head16 = (size_t)12568 * 4 * 768 * 2 / 16;
    __shared__ i64 x[PP_ROW];
    __shared__ i64 red[4];
    const int tid = threadIdx.x, b = blockIdx.x;
    const long long t0 = (long long)__builtin_amdgcn_s_memrealtime();
    unsigned seq = 0;
    int word = 0;
    v4i wq[4], wp[2], wf[5], wm[5];
    pp_fetch<4>(wq, a.plates, qkvB / 16);                  // layer 0's qkv share (each later one: before its wait)
    for (int step = 0; step < a.steps; step++) {
        // the entering row: every block reads the word's row itself (no hand-off)
        for (int i = tid; i < 768; i += 256) x[i] = a.wte[(size_t)(word % 1024) * 768 + i] + step;
        __syncthreads();
        if (step == a.steps - 1 && b == 0 && tid == 0) a.stamps[0] = (long long)__builtin_amdgcn_s_memrealtime();
        for (int l = 0; l < 12; l++) {
            const v4i* pq = a.plates + (size_t)l * layer16;
            const v4i* pp = pq + qkvB / 16;
            const v4i* pf = pp + projB / 16;
            const v4i* pm = pf + fcB / 16;
            // qkv: the row (in x), the plate share (requested before the row's wait), 9 outputs a block
            pp_fetch<2>(wp, pp, projB / 16);               // (proj's share, ahead of the waits below)
            i64 s = pp_rowsum(x, 768, red) + pp_fold<4>(wq);
            for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            seq++;
            const unsigned tq = seq;
            if (tid < 9) pp_put(a.rows, 0, b * 9 + tid, tq, s + tid);
            // attention: blocks 0-11 take their head's q, k, v entries and its cached positions
            seq++;
            const unsigned ta = seq;
            if (b < 12) {
                const int h = b;
                if (!pp_get<1>(a, 0, h * 64, 64, tq, x, t0) || !pp_get<1>(a, 0, 768 + h * 64, 64, tq, x + 64, t0) ||
                    !pp_get<1>(a, 0, 1536 + h * 64, 64, tq, x + 128, t0))
                    return;
                if (tid < 64) {
                    const size_t kv = ((size_t)l * 12 + h) * a.ctx * 64;
                    i64 o = x[tid] ^ x[64 + tid] ^ x[128 + tid];
                    for (int r = 0; r < a.P; r++) o += a.K[kv + r * 64 + tid] + a.V[kv + r * 64 + tid];
                    pp_put(a.rows, 1, h * 64 + tid, ta, o);
                }
                __syncthreads();                           // (x is read above before the next wait refills it)
            }
            // proj: the attention row, 3 outputs a block
            pp_fetch<5>(wf, pf, fcB / 16);                 // (fc's share, ahead of the wait)
            const int sb = step == a.steps - 1 ? 1 + l * 5 : -100;
            if (!pp_get<3>(a, 1, 0, 768, ta, x, t0, sb + 0)) return;
            s = pp_rowsum(x, 768, red) + pp_fold<2>(wp);
            seq++;
            const unsigned tp = seq;
            if (tid < 3) pp_put(a.rows, 2, b * 3 + tid, tp, s + tid);
            // fc: the stream row, 12 outputs a block
            pp_fetch<5>(wm, pm, mpB / 16);                 // (mproj's share, ahead of the wait)
            if (!pp_get<3>(a, 2, 0, 768, tp, x, t0, sb + 1)) return;
            s = pp_rowsum(x, 768, red) + pp_fold<5>(wf);
            seq++;
            const unsigned tf = seq;
            if (tid < 12) pp_put(a.rows, 3, b * 12 + tid, tf, s + tid);
            // mproj: the hidden row (3072), 3 outputs a block
            if (!pp_get<12>(a, 3, 0, 3072, tf, x, t0, sb + 2)) return;
            s = pp_rowsum(x, 3072, red) + pp_fold<5>(wm);
            seq++;
            const unsigned tm = seq;
            if (tid < 3) pp_put(a.rows, 4, b * 3 + tid, tm, s + tid);
            if (l < 11) pp_fetch<4>(wq, pm + mpB / 16, qkvB / 16);   // the next layer's qkv share, before the wait
            if (!pp_get<3>(a, 4, 0, 768, tm, x, t0, sb + 3)) return;   // the next layer's (or the head's) row
        }
        // the head: the stream row is in x; the block's 1/256 of the word table, its best
        {
            const v4i* ph = a.plates + (size_t)12 * layer16;
            const size_t share = (head16 + PP_NB - 1) / PP_NB, b0 = (size_t)b * share;
            i64 best = pp_rowsum(x, 768, red);
            const size_t end = std::min(b0 + share, head16);
            for (size_t i0 = b0 + tid; i0 < end; i0 += 256 * 8) {      // eight loads in flight a thread
                v4i w[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const size_t i = i0 + 256 * k;
                    w[k] = ph[i < end ? i : b0];
                }
#pragma unroll
                for (int k = 0; k < 8; k++) best += w[k].x ^ w[k].y ^ w[k].z ^ w[k].w;
            }
            for (int o = 32; o > 0; o >>= 1) best = max(best, __shfl_xor(best, o, 64));
            if ((tid & 63) == 0) red[tid >> 6] = best;
            __syncthreads();
            best = max(max(red[0], red[1]), max(red[2], red[3]));
            __syncthreads();
            seq++;
            if (tid == 0) pp_put(a.rows, 5, b, seq, best);
            if (step == a.steps - 1 && b == 0 && tid == 0) a.stamps[61] = (long long)__builtin_amdgcn_s_memrealtime();
            // the race in every block: the 256 bests (the next step's first qkv share requested before the wait)
            pp_fetch<4>(wq, a.plates, qkvB / 16);
            if (!pp_get<1>(a, 5, 0, PP_NB, seq, x, t0, step == a.steps - 1 ? 62 : -1)) return;
            i64 w = 0;
            for (int i = tid; i < PP_NB; i += 256) w = max(w, x[i]);
            for (int o = 32; o > 0; o >>= 1) w = max(w, __shfl_xor(w, o, 64));
            if ((tid & 63) == 0) red[tid >> 6] = w;
            __syncthreads();
            word = (int)((unsigned long long)max(max(red[0], red[1]), max(red[2], red[3])) & 1023);
            __syncthreads();
        }
    }
    if (tid == 0) a.sink[b] = word;
}

static int run_persist(double& us, int& late) {
    const size_t qkvB = 768 * 2304 * 2, projB = 768 * 768 * 2, fcB = 768 * 3072 * 2, mpB = 3072 * 768 * 2;
    const size_t headB = (size_t)12568 * 4 * 768 * 2, layerB = qkvB + projB + fcB + mpB;
    const int CTX = 64, P = 16, WTE = 1024, STEPS = 15, REPS = 20;
    int dev = 0, cus = 0, coop = 0;
    CHK(hipGetDevice(&dev));
    CHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    CHK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    int per_cu = 0;
    CHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k_persist, 256, 0));
    if (!coop || per_cu * cus < PP_NB) { fprintf(stderr, "floor_probe: 256 co-resident blocks not available\n"); us = -1; return 0; }
    char* plates = nullptr;
    unsigned long long* rows;
    short* K;
    int *V, *err;
    i64 *wte, *sink;
    CHK(hipMalloc(&plates, 12 * layerB + headB));
    CHK(hipMalloc(&rows, (size_t)PP_SLOTS * PP_ROW * 16));
    CHK(hipMalloc(&K, (size_t)12 * 12 * CTX * 64 * 2)); CHK(hipMalloc(&V, (size_t)12 * 12 * CTX * 64 * 4));
    CHK(hipMalloc(&wte, (size_t)WTE * 768 * 8)); CHK(hipMalloc(&sink, PP_NB * 8)); CHK(hipMalloc(&err, 4));
    long long* stamps;
    CHK(hipMalloc(&stamps, 64 * 8)); CHK(hipMemset(stamps, 0, 64 * 8));
    CHK(hipMemset(plates, 1, 12 * layerB + headB)); CHK(hipMemset(rows, 0, (size_t)PP_SLOTS * PP_ROW * 16));
    CHK(hipMemset(K, 0, (size_t)12 * 12 * CTX * 64 * 2)); CHK(hipMemset(V, 0, (size_t)12 * 12 * CTX * 64 * 4));
    CHK(hipMemset(wte, 0, (size_t)WTE * 768 * 8)); CHK(hipMemset(err, 0, 4));
    CHK(hipDeviceSynchronize());
    hipStream_t st;
    CHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    PersistArgs a{};
    a.plates = (const v4i*)plates; a.rows = rows; a.K = K; a.V = V; a.wte = wte; a.err = err; a.sink = sink; a.stamps = stamps;
    a.steps = STEPS; a.ctx = CTX; a.P = P; a.limit = 20000000;     // 0.2 s
    void* args[] = {&a};
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0)); CHK(hipEventCreate(&e1));
    // every launch starts its sequence numbers at 1 again: the rows are emptied between launches
    auto once = [&]() -> int {
        CHK(hipMemsetAsync(rows, 0, (size_t)PP_SLOTS * PP_ROW * 16, st));
        CHK(hipEventRecord(e0, st));
        CHK(hipLaunchCooperativeKernel((const void*)k_persist, dim3(PP_NB), dim3(256), args, 0, st));
        CHK(hipEventRecord(e1, st));
        CHK(hipStreamSynchronize(st));
        return 0;
    };
    double best = 1e30;
    for (int r = 0; r < 3 + REPS; r++) {
        if (once()) return 1;
        float ms = 0.0f;
        CHK(hipEventElapsedTime(&ms, e0, e1));
        if (r >= 3) best = std::min(best, ms * 1000.0 / STEPS);
        CHK(hipMemcpy(&late, err, 4, hipMemcpyDeviceToHost));
        if (late) break;
    }
    us = best;
    long long h[64];
    CHK(hipMemcpy(h, stamps, sizeof(h), hipMemcpyDeviceToHost));
    fprintf(stderr, "phase ends (us from the step's start, block 0, the last step):");
    for (int i = 1; i < 63; i++) if (h[i]) fprintf(stderr, " %d:%.2f", i, (h[i] - h[0]) / 100.0);
    fprintf(stderr, "\n");
    CHK(hipFree(stamps));
    CHK(hipEventDestroy(e0)); CHK(hipEventDestroy(e1)); CHK(hipStreamDestroy(st));
    for (void* q : {(void*)plates, (void*)rows, (void*)K, (void*)V, (void*)wte, (void*)sink, (void*)err}) CHK(hipFree(q));
    return 0;
}

// ---- the Pythia machine at 32 streams ----
// a paired launch: blocks [0, na) read NA1 int4 a thread of A (the attention: its (head, stream)'s cache rows), the
// rest NA2 of B and NB2 of C (mproj's partials: the tile's hidden rows and three column tiles)
template <int NA1, int NA2, int NB2, bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_pair(const v4i* A, size_t ra, int na, const v4i* B, const v4i* C, size_t rc, i64* out) {
    if (EMPTY) return;
    const int tid = threadIdx.x, b = blockIdx.x;
    int s = 0;
    if (b < na) {
        const v4i* a = A + (size_t)b * ra + tid;
#pragma unroll
        for (int i = 0; i < NA1; i++) { const v4i v = a[256 * i]; s += v.x ^ v.w; }
    } else {
        const v4i* x = B + tid;
        const v4i* c = C + (size_t)((b - na) % 64) * rc + tid;      // 64 column groups, each read by both row tiles
#pragma unroll
        for (int i = 0; i < NA2; i++) { const v4i v = x[256 * i]; s += v.x ^ v.w; }
#pragma unroll
        for (int i = 0; i < NB2; i++) { const v4i v = c[256 * i]; s += v.x ^ v.w; }
    }
    for (int i = tid; i < 64; i += 256) out[(size_t)b * 64 + i] = s + i;
}

template <bool EMPTY>
static int runpy(double& us) {
    const size_t qkvB = 768 * 2304 * 2, projB = 768 * 768 * 2, fcB = 768 * 3072 * 2, mpB = 3072 * 768 * 2;
    const size_t headB = (size_t)768 * 50304 * 2, layerB = qkvB + projB + fcB + mpB;
    const size_t kvL = (size_t)32 * 12 * 320 * 396;          // a layer's cache: 32 streams x 12 heads x 320 positions
    const size_t planesB = 2 * 36864 * 2, rowsB = (size_t)32 * 3072 * 8, NOUTV = 1 << 19;
    const int STEPS = 16, REPS = 10;
    char *plates = nullptr, *planes, *rows, *kv;
    i64* out;
    CHK(hipMalloc(&plates, 12 * layerB + headB)); CHK(hipMalloc(&planes, planesB)); CHK(hipMalloc(&rows, rowsB));
    CHK(hipMalloc(&kv, 12 * kvL)); CHK(hipMalloc(&out, NOUTV * 8));
    CHK(hipMemset(plates, 1, 12 * layerB + headB)); CHK(hipMemset(planes, 1, planesB)); CHK(hipMemset(rows, 1, rowsB));
    CHK(hipMemset(kv, 1, 12 * kvL)); CHK(hipMemset(out, 0, NOUTV * 8));
    CHK(hipDeviceSynchronize());
    hipStream_t st;
    CHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    const v4i *P = (const v4i*)planes, *Rw = (const v4i*)rows;
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int s = 0; s < STEPS; s++) {
        const char* pl = plates;
        // the words enter: a row a block
        k_floor_move<192, 2, 0, 288, EMPTY, 8><<<dim3(1, 32), 192, 0, st>>>(Rw, 384, 0, Rw, 0, out);
        for (int l = 0; l < 12; l++) {
            const v4i* wq = (const v4i*)pl; pl += qkvB + projB;           // qkv, proj, fc contiguous
            pl += fcB;
            const v4i* wm = (const v4i*)pl; pl += mpB;
            const v4i* kvl = (const v4i*)(kv + l * kvL);
            // fc | qkv: 336 column tiles x 2 row tiles, each its light planes (36 KB) and its plate tile (24 KB)
            k_floor_move<256, 9, 6, 256, EMPTY, 11><<<dim3(336, 2), 256, 0, st>>>(P, 2304, 0, wq, 1536, out);
            // the attention (384 blocks, 192 positions of cache rows: 76 KB) | mproj partials (128 blocks: the tile's
            // hidden rows at 32 bits, 48 KB, and three column tiles, 72 KB)
            k_floor_pair<19, 12, 18, EMPTY><<<512, 256, 0, st>>>(kvl, 4752, 384, Rw, wm, 4608, out);
            // proj: the attention rows at 32 bits (48 KB), its plate tile (24 KB), mproj's partials for its tile (8 KB)
            k_floor_move<256, 14, 6, 256, EMPTY, 12><<<dim3(48, 2), 256, 0, st>>>(Rw, 3072, 0, wq + (qkvB / 16), 1536, out);
            // the row kernel: the stream row, both gauges' planes
            k_floor_move<192, 2, 0, 576, EMPTY, 13><<<dim3(1, 32), 192, 0, st>>>(Rw, 384, 0, Rw, 0, out);
        }
        k_floor_head64<EMPTY, 12><<<512, 256, 0, st>>>(P, (const v4i*)pl, headB / 16, out);
        if (s == STEPS - 1) k_floor_race64<EMPTY><<<32, 256, 0, st>>>(out, out + (1 << 18));
    }
    CHK(hipStreamEndCapture(st, &g));
    CHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    hipEvent_t e0, e1;
    CHK(hipEventCreate(&e0)); CHK(hipEventCreate(&e1));
    for (int i = 0; i < 2; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipStreamSynchronize(st));
    CHK(hipEventRecord(e0, st));
    for (int i = 0; i < REPS; i++) CHK(hipGraphLaunch(ge, st));
    CHK(hipEventRecord(e1, st));
    CHK(hipStreamSynchronize(st));
    float ms = 0.0f;
    CHK(hipEventElapsedTime(&ms, e0, e1));
    us = ms * 1000.0 / (REPS * STEPS);
    CHK(hipEventDestroy(e0)); CHK(hipEventDestroy(e1));
    CHK(hipGraphExecDestroy(ge)); CHK(hipGraphDestroy(g)); CHK(hipStreamDestroy(st));
    for (void* q : {(void*)plates, (void*)planes, (void*)rows, (void*)kv, (void*)out}) CHK(hipFree(q));
    return 0;
}

int main(int argc, char** argv) {
    if (argc > 1 && std::string(argv[1]) == "persist") {
        double us = 0;
        int late = 0;
        if (run_persist(us, late)) return 1;
        printf("{\"persist_us\": %.2f, \"late\": %d, \"handoffs\": 61, \"graph_steps\": 15}\n", us, late);
        return 0;
    }
    double empty = 1e30, bytes = 1e30, e64 = 1e30, b64 = 1e30, epy = 1e30, bpy = 1e30;
    for (int r = 0; r < 3; r++) {             // the best of three measurements of each form
        double e, b;
        if (run<true>(e) || run<false>(b)) return 1;
        empty = e < empty ? e : empty;
        bytes = b < bytes ? b : bytes;
        if (run64<true>(e) || run64<false>(b)) return 1;
        e64 = e < e64 ? e : e64;
        b64 = b < b64 ? b : b64;
        if (runpy<true>(e) || runpy<false>(b)) return 1;
        epy = e < epy ? e : epy;
        bpy = b < bpy ? b : bpy;
    }
    printf("{\"launches\": 61.07, \"empty_us\": %.2f, \"bytes_us\": %.2f, \"ctx\": 16, \"graph_steps\": 15, "
           "\"b64\": {\"launches\": 86, \"empty_us\": %.2f, \"bytes_us\": %.2f, \"ctx\": 96, \"graph_steps\": 16}, "
           "\"pythia32\": {\"launches\": 50.06, \"empty_us\": %.2f, \"bytes_us\": %.2f, \"ctx\": 192, \"graph_steps\": 16}}\n",
           empty, bytes, e64, b64, epy, bpy);
    return 0;
}
