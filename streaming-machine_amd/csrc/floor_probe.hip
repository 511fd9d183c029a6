// The decode step's launch-structure floor, measured.  Batch 1: the step's 62 dependent launches (12 layers x
// [qkv, attend, proj, fc, mproj], the head, the race) with the machine's grids and block sizes,
// replayed from a HIP graph of 15 steps, in two forms:
//   empty  - every kernel returns at once: the cost of 62 dependent launches alone;
//   bytes  - every kernel reads the row it depends on (the previous kernel's output) and its share of its plate
//            (the GPT-2 124M shapes: int16 plates of 768x2304, 768x768, 768x3072, 3072x768, and the 768 x 50257
//            word table, read whole as the machine's default head does), the attention reads 16 cached positions
//            of keys (int16) and values
//            (int32) per head, and each kernel writes its outputs -- no arithmetic beyond folding what it read.
// The machine's step does all of this plus its arithmetic, so its time over "bytes" is what the arithmetic,
// the block reductions and the table reads cost.
// 64 streams ("b64"): the batched step's 86 launches (12 layers x [qkv, attend, proj, light, fc, mproj
// partials, light], the head, the race) with the machine's grids, graphs of 16 steps, the same two forms; in
// "bytes" each bank block reads its row tile's light planes or int32 rows and its plate share, each attention
// block 96 positions of its cache rows (38 KB), each light block its row (and the partials), the head its plate.
// Prints one JSON line with both.
#include <hip/hip_runtime.h>
#include <cstdio>

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
            k_floor_phase<768, 2, 4, 2, EMPTY><<<288, 256, 0, st>>>(R, wq, 1152, QKV);
            k_floor_attend<EMPTY><<<12, 256, 0, st>>>(QKV, K + kv, V + kv, P, CTX, att);
            k_floor_phase<768, 2, 2, 2, EMPTY><<<192, 128, 0, st>>>(att, wp, 384, R);
            k_floor_phase<768, 2, 4, 2, EMPTY><<<384, 256, 0, st>>>(R, wf, 1536, hid);
            k_floor_phase<3072, 1, 4, 2, EMPTY><<<192, 256, 0, st>>>(hid, wm, 768, R);
        }
        k_floor_phase<768, 4, 4, 2, EMPTY, true><<<512, 256, 0, st>>>(R, (const v4i*)pl, head_tiles, part);
        k_floor_race<EMPTY><<<1, 256, 0, st>>>(part, 512, wte, WTE, R);
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
// the head: each block its waves' light planes, then its share of the plate
template <bool EMPTY>
__global__ __launch_bounds__(256) void k_floor_head64(const v4i* planes, const v4i* W, size_t nW, i64* part) {
    if (EMPTY) return;
    const int tid = threadIdx.x;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 24; i++) { const v4i v = planes[tid + 256 * i]; s += v.x ^ v.y; }
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

int main() {
    double empty = 1e30, bytes = 1e30, e64 = 1e30, b64 = 1e30;
    for (int r = 0; r < 3; r++) {             // the best of three measurements of each form
        double e, b;
        if (run<true>(e) || run<false>(b)) return 1;
        empty = e < empty ? e : empty;
        bytes = b < bytes ? b : bytes;
        if (run64<true>(e) || run64<false>(b)) return 1;
        e64 = e < e64 ? e : e64;
        b64 = b < b64 ? b : b64;
    }
    printf("{\"launches\": 62, \"empty_us\": %.2f, \"bytes_us\": %.2f, \"ctx\": 16, \"graph_steps\": 15, "
           "\"b64\": {\"launches\": 86, \"empty_us\": %.2f, \"bytes_us\": %.2f, \"ctx\": 96, \"graph_steps\": 16}}\n",
           empty, bytes, e64, b64);
    return 0;
}
