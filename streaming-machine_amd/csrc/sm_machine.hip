// Host side of libsm_base2.so: the C ABI of include/sm_base2.h.
//
// One machine = one HIP stream, the device image of a base2_gpu.py directory, the per-layer integer KV
// cache and a few control words on the device (position, prompt length, error bits).  A decode step is the
// launch sequence
//     for each of the 12 layers:  qkv (gauge + product + gauged)  ->  attention  ->  proj (to16 + product +
//                                 plain, added to the stream)  ->  fc (gauge + product + gauged + edge)  ->
//                                 mproj (to16 + product + plain, added)
//     head (gauge + product + gauged + standing amount + race; the word goes straight back into seq)
// i.e. 61 launches with the device-side position advancing in the head, so a captured HIP graph of
// graph_steps consecutive steps replays the loop; the host synchronises once per sm_generate call
// (base2_stream.swift:273-281 commits one command buffer per prompt the same way).
#include "sm_kernels.hip"
#include "sm_batch.hip"
#include "sm_attend_split.hip"
#include "../../include/sm_base2.h"

#include <hip/hip_ext.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <atomic>
#include <cstdlib>
#include <cxxabi.h>
#include <map>
#include <mutex>
#include <string>
#include <vector>

static thread_local std::string g_err;

// the batch-1 machine's default split position (sm_config.att_split = 0): from this position on a step's attention
// runs spread over chunks of 64 positions (sm_attend_split.hip), below it one block a head (k_attend)
#define SM_ATT_SPLIT_AT 160

static int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(x)                                                                                   \
    do {                                                                                             \
        hipError_t e_ = (x);                                                                         \
        if (e_ != hipSuccess) return fail(SM_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)

extern "C" const char* sm_last_error(void) { return g_err.c_str(); }

// ---------------------------------------------------------------------------------------------------------
// Kernel timing.  A machine created with profile = 1 (its launches) and, after sm_profile_stages(1), the stage and
// plate entry points stamp every launch with a HIP event pair by its own dispatch (hipExtLaunchKernelGGL on the
// launching stream: the interval a kernel trace reports); sm_profile_kernels folds the pairs into launches and
// summed microseconds per kernel name.  Launches that are not timed pass null events.
struct KernelTiming {
    std::mutex mu;
    std::atomic<bool> stages{false};   // read by every stage launch without the lock
    std::vector<std::string> names;
    std::vector<long long> n;
    std::vector<double> us;
    // per name: timed launches by kernel symbol (the demangled device function, as a kernel trace names it)
    std::vector<std::map<std::string, long long>> syms;
    std::map<const void*, std::string> symbol_of;
    struct Pend { int id; hipEvent_t s, e; };
    std::vector<Pend> pend;
    std::vector<hipEvent_t> spare;
};
static KernelTiming g_kt;

static int kt_id(const char* name) {                 // (g_kt.mu held)
    for (size_t i = 0; i < g_kt.names.size(); i++)
        if (g_kt.names[i] == name) return (int)i;
    g_kt.names.push_back(name);
    g_kt.n.push_back(0);
    g_kt.us.push_back(0.0);
    g_kt.syms.emplace_back();
    return (int)g_kt.names.size() - 1;
}
static const std::string& kt_symbol(const void* kernel, hipStream_t st) {   // (g_kt.mu held)
    auto it = g_kt.symbol_of.find(kernel);
    if (it != g_kt.symbol_of.end()) return it->second;
    std::string sym = "?";
    if (const char* raw = hipKernelNameRefByPtr(kernel, st)) {
        int status = 0;
        char* dm = abi::__cxa_demangle(raw, nullptr, nullptr, &status);
        sym = status == 0 && dm ? dm : raw;
        std::free(dm);
    }
    return g_kt.symbol_of.emplace(kernel, sym).first->second;
}
static hipEvent_t kt_event() {                       // (g_kt.mu held)
    hipEvent_t e = nullptr;
    if (!g_kt.spare.empty()) {
        e = g_kt.spare.back();
        g_kt.spare.pop_back();
    } else if (hipEventCreate(&e) != hipSuccess) {
        e = nullptr;
    }
    return e;
}

template <typename F, typename... A>
static void launch(bool timed, const char* name, F kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t st, A... args) {
    hipEvent_t s = nullptr, e = nullptr;
    if (timed) {
        std::lock_guard<std::mutex> lock(g_kt.mu);
        s = kt_event();
        e = kt_event();
        if (s && e) {
            const int id = kt_id(name);
            g_kt.syms[id][kt_symbol(reinterpret_cast<const void*>(kernel), st)]++;
            g_kt.pend.push_back({id, s, e});
        } else {
            if (s) g_kt.spare.push_back(s);
            if (e) g_kt.spare.push_back(e);
            s = e = nullptr;
        }
    }
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)shmem, st, s, e, 0u, args...);
}

// every pending pair, once the device has finished them, into the per-name sums
static int kt_fold() {
    HIP_TRY(hipDeviceSynchronize());
    std::lock_guard<std::mutex> lock(g_kt.mu);
    for (const auto& p : g_kt.pend) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, p.s, p.e) != hipSuccess) return fail(SM_E_HIP, "hipEventElapsedTime");
        g_kt.n[p.id]++;
        g_kt.us[p.id] += 1000.0 * ms;
        g_kt.spare.push_back(p.s);
        g_kt.spare.push_back(p.e);
    }
    g_kt.pend.clear();
    return SM_OK;
}

// ---------------------------------------------------------------------------------------------------------
// plates
struct DevPlate {
    int nin = 0, nout = 0, tc = 0, ntiles = 0;
    int16_t* W = nullptr;
    int* e = nullptr;
    i64* b = nullptr;
    i64* sw = nullptr;      // the complement machine: each column's sum over the plain plate (W then holds ~w)
    int16_t* W2 = nullptr;  // split digits (MODE_SPLIT): the subtracted plate, tiled as W (the digit is W - W2)
};

// input-major [nin][nout] -> column tiles of tc: unit u of tile t holds inputs 8 (u / tc) .. + 8 of column
// t tc + u % tc (padding columns are zero)
static std::vector<int16_t> tile_plate(const int16_t* w, int nin, int nout, int tc) {
    const int ntiles = (nout + tc - 1) / tc;
    std::vector<int16_t> t((size_t)ntiles * tc * nin, 0);
    for (int k = 0; k < nin; k++) {
        const int16_t* row = w + (size_t)k * nout;
        const size_t kb = (size_t)(k / 8) * tc * 8 + (k % 8);
        for (int j = 0; j < nout; j++) {
            const int tile = j / tc, jj = j % tc;
            t[(size_t)tile * tc * nin + kb + (size_t)jj * 8] = row[j];
        }
    }
    return t;
}

static void hfree(void* p) {
    if (p) (void)hipFree(p);
}

template <typename T>
static int dalloc(T** p, size_t count) {
    if (count == 0) count = 1;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess) return fail(SM_E_OOM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return SM_OK;
}

// inv: the plate held complemented, with its plain column sums (base2_stream.swift:189-190); w2 (split digits):
// the subtracted plate, tiled as w
static int upload_plate(DevPlate& P, const int16_t* w, const int32_t* e, const i64* b, int nin, int nout, int tc,
                        bool inv = false, const int16_t* w2 = nullptr) {
    if (nin % 8 || nin <= 0 || nout <= 0 || (tc != 1 && tc != 2 && tc != 4 && tc != 8))
        return fail(SM_E_ARG, "plate: nin must be a multiple of 8 and tile_cols one of 1, 2, 4, 8");
    P.nin = nin; P.nout = nout; P.tc = tc; P.ntiles = (nout + tc - 1) / tc;
    std::vector<int16_t> t = tile_plate(w, nin, nout, tc);
    int rc;
    if ((rc = dalloc(&P.W, t.size())) || (rc = dalloc(&P.e, (size_t)nout)) || (rc = dalloc(&P.b, (size_t)nout))) return rc;
    if (inv) {
        std::vector<i64> sw((size_t)nout, 0);
        for (int k = 0; k < nin; k++)
            for (int j = 0; j < nout; j++) sw[j] += w[(size_t)k * nout + j];
        for (auto& x : t) x = (int16_t)~x;
        if ((rc = dalloc(&P.sw, (size_t)nout))) return rc;
        HIP_TRY(hipMemcpy(P.sw, sw.data(), (size_t)nout * 8, hipMemcpyHostToDevice));
    }
    HIP_TRY(hipMemcpy(P.W, t.data(), t.size() * 2, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(P.e, e, (size_t)nout * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(P.b, b, (size_t)nout * 8, hipMemcpyHostToDevice));
    if (w2) {
        const std::vector<int16_t> t2 = tile_plate(w2, nin, nout, tc);
        if ((rc = dalloc(&P.W2, t2.size()))) return rc;
        HIP_TRY(hipMemcpy(P.W2, t2.data(), t2.size() * 2, hipMemcpyHostToDevice));
    }
    return SM_OK;
}

// the top read's high-byte plane in column tiles of tc: unit u of tile t holds inputs 16 (u / tc) .. + 16 of
// column t tc + u % tc, each as w >> 8 (padding columns zero); and its low bytes w & 255, word by word
static std::vector<int8_t> tile_hi_plane(const int16_t* w, int nin, int nout, int tc) {
    const int ntiles = (nout + tc - 1) / tc;
    std::vector<int8_t> t((size_t)ntiles * tc * nin, 0);
    for (int k = 0; k < nin; k++) {
        const int16_t* row = w + (size_t)k * nout;
        const size_t kb = (size_t)(k / 16) * tc * 16 + (k % 16);
        for (int j = 0; j < nout; j++) t[(size_t)(j / tc) * tc * nin + kb + (size_t)(j % tc) * 16] = (int8_t)(row[j] >> 8);
    }
    return t;
}
static std::vector<uint8_t> lo_plane(const int16_t* w, int nin, int nout) {
    std::vector<uint8_t> t((size_t)nout * nin);
    for (int k = 0; k < nin; k++)
        for (int j = 0; j < nout; j++) t[(size_t)j * nin + k] = (uint8_t)(w[(size_t)k * nout + j] & 255);
    return t;
}

static void free_plate(DevPlate& P) {
    hfree(P.W); hfree(P.e); hfree(P.b); hfree(P.sw); hfree(P.W2);
    P = DevPlate();
}

// Byte planes for the MFMA path: column tiles of 16, 64-k steps, planes wh and wl' = (w & 255) - 128, in the
// MFMA B-operand order (lane l: column l % 16, bytes k = 16 (l / 16) + b); plus each column's plane sums.
struct MfmaPlate {
    int K = 0, N = 0, ntiles = 0;
    signed char* W = nullptr;
    int* csum = nullptr;
    int* e = nullptr;
    i64* b = nullptr;
};

static int upload_mfma_plate(MfmaPlate& P, const int16_t* w, const int32_t* e, const i64* b, int K, int N) {
    if (K % 64 || N <= 0) return fail(SM_E_ARG, "mfma plate: K must be a multiple of 64");
    const int KS = K / 64, nt = (N + 15) / 16;
    P.K = K; P.N = N; P.ntiles = nt;
    std::vector<signed char> out((size_t)nt * KS * 2 * 1024, 0);
    std::vector<int> cs((size_t)N * 2, 0);
    for (int k = 0; k < K; k++) {
        const int16_t* row = w + (size_t)k * N;
        const int s = k >> 6, kk = k & 63, g = kk >> 4, bb = kk & 15;
        for (int col = 0; col < N; col++) {
            const int v = row[col], wh = v >> 8, wl = (v & 255) - 128;
            const size_t base = ((size_t)((col >> 4) * KS + s) * 2) * 1024 + (size_t)((col & 15) + 16 * g) * 16 + bb;
            out[base] = (signed char)wh;
            out[base + 1024] = (signed char)wl;
            cs[2 * col] += wh;
            cs[2 * col + 1] += wl;
        }
    }
    int rc;
    if ((rc = dalloc(&P.W, out.size())) || (rc = dalloc(&P.csum, cs.size())) || (rc = dalloc(&P.e, (size_t)N)) ||
        (rc = dalloc(&P.b, (size_t)N)))
        return rc;
    HIP_TRY(hipMemcpy(P.W, out.data(), out.size(), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(P.csum, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(P.e, e, (size_t)N * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(P.b, b, (size_t)N * 8, hipMemcpyHostToDevice));
    return SM_OK;
}

static void free_mfma_plate(MfmaPlate& P) {
    hfree(P.W); hfree(P.csum); hfree(P.e); hfree(P.b);
    P = MfmaPlate();
}

// ---------------------------------------------------------------------------------------------------------
// tables
struct sm_tables {
    int* LOG2 = nullptr; int* EXP2 = nullptr; int* PHI = nullptr; int* ARR = nullptr;
    int* GPOW = nullptr; int* HPOW = nullptr; int* PGPOW = nullptr;
    int alen = 0;
    i64 log768 = 0, eps40 = 0;
    int verified = 0;         // every entry equals its defining formula (checked on the device at create)
    int* scratch = nullptr;   // [0] pos for sm_stage_attend, [1] error bits, [4..7] mismatch counts
    // sm_stage_attend_split's score row, chunk maxima and accumulators (made at its first call, for ctx <= 8192)
    i64 *asc = nullptr, *acm = nullptr, *aacc = nullptr;
    Tables tb() const { return Tables{LOG2, EXP2, PHI, ARR, alen, log768, eps40, GPOW, HPOW, PGPOW}; }
};

static int upload_table(int** dst, const i64* src, size_t n, i64 lo, i64 hi, const char* name) {
    std::vector<int> v(n);
    for (size_t i = 0; i < n; i++) {
        if (src[i] < lo || src[i] > hi) return fail(SM_E_IO, std::string("table ") + name + " value out of range");
        v[i] = (int)src[i];
    }
    int rc = dalloc(dst, n);
    if (rc) return rc;
    HIP_TRY(hipMemcpy(*dst, v.data(), n * 4, hipMemcpyHostToDevice));
    return SM_OK;
}

static int tables_init(sm_tables& T, const i64* phi, const i64* arr, int alen, const i64* log2t, const i64* exp2t,
                       i64 log768, i64 eps40) {
    if (alen <= 0 || alen > (1 << 20)) return fail(SM_E_ARG, "arrival table length");
    int rc;
    if ((rc = upload_table(&T.PHI, phi, 65536, 0, 65536, "phi"))) return rc;
    if ((rc = upload_table(&T.ARR, arr, alen, 0, 1 << 24, "arrival"))) return rc;
    if ((rc = upload_table(&T.LOG2, log2t, 65536, 0, 65536, "log2"))) return rc;
    if ((rc = upload_table(&T.EXP2, exp2t, 65536, 65536, 131072, "exp2"))) return rc;
    // derived tables: exact integer compositions of LOG2 and EXP2 (see Tables in sm_device.h)
    {
        std::vector<i64> g(2 * 65536), pg(2 * 65536), hp(65536);
        for (int r = 0; r < 2; r++)
            for (int m = 0; m < 65536; m++) {
                g[r * 65536 + m] = exp2t[(log768 - (((i64)r * 65536 + log2t[m]) >> 1)) & 0xFFFF];
                pg[r * 65536 + m] = exp2t[(-(((i64)r * 65536 + log2t[m]) >> 1)) & 0xFFFF];
            }
        for (int m = 0; m < 65536; m++) hp[m] = exp2t[(-log2t[m]) & 0xFFFF];
        if ((rc = upload_table(&T.GPOW, g.data(), g.size(), 65536, 131072, "gauge power")) ||
            (rc = upload_table(&T.PGPOW, pg.data(), pg.size(), 65536, 131072, "Pythia gauge power")) ||
            (rc = upload_table(&T.HPOW, hp.data(), hp.size(), 65536, 131072, "arrival divisor")))
            return rc;
    }
    if ((rc = dalloc(&T.scratch, 16))) return rc;
    HIP_TRY(hipMemset(T.scratch, 0, 64));
    T.alen = alen; T.log768 = log768; T.eps40 = eps40;
    // every entry against its formula (table_mode 1 refuses tables that are not the reference's)
    const int n = alen + 1 > 65536 ? alen + 1 : 65536;
    k_check_tables<<<(n + 255) / 256, 256>>>(T.tb(), reinterpret_cast<unsigned*>(T.scratch + 4));
    HIP_TRY(hipGetLastError());
    unsigned bad[4];
    HIP_TRY(hipMemcpy(bad, T.scratch + 4, sizeof(bad), hipMemcpyDeviceToHost));
    T.verified = (bad[0] | bad[1] | bad[2] | bad[3]) == 0;
    return SM_OK;
}

static void tables_free(sm_tables& T) {
    hfree(T.LOG2); hfree(T.EXP2); hfree(T.PHI); hfree(T.ARR); hfree(T.GPOW); hfree(T.HPOW); hfree(T.PGPOW); hfree(T.scratch);
    hfree(T.asc); hfree(T.acm); hfree(T.aacc);
    T = sm_tables();
}

// ---------------------------------------------------------------------------------------------------------
// the machine
// CTL_POS / CTL_POS1: the position's two slots.  A step reads the slot of the machine's parity; a race run as
// part of another kernel's blocks (the race of the step before folded into a step's first kernel, and every
// batched race) writes the next position into the other slot, which no block of that kernel reads, so the race
// needs no grid-wide handoff (a last-arriving block behind a fence costs more than the kernel boundary it would
// save).  Batch 1's k_race1 (one block, a run's last step, and the machines that do not fold) advances its slot in
// place
enum { CTL_POS = 0, CTL_PLEN = 1, CTL_NWORDS = 2, CTL_ERR = 3, CTL_RECPOS = 4, CTL_POS1 = 6, CTL_N = 8 };
static const int NIN[4] = {768, 768, 768, 3072};
static const int NOUT[4] = {2304, 768, 3072, 768};
static const int TCOLS[4] = {2, 2, 2, 1};      // tile widths: qkv, proj, fc, mproj (one wave per tile)
static const char* BANK[4] = {"qkv", "proj", "fc", "mproj"};

struct sm_machine {
    sm_config cfg{};
    int B = 1, ctx = 0, vocab = 0, npos = 0, head_grid = 1024;
    int RC = 1;                    // rows the MFMA phases hold: the streams, or a pass of prompt rows
    hipStream_t st = nullptr;
    DevPlate bank[12][4];          // batch 1: GEMV tiles
    DevPlate head;
    MfmaPlate mbank[12][4];        // batched streams: MFMA byte planes
    MfmaPlate mhead;
    signed char* planes = nullptr;  // [4][48][3][1024] light planes of the current phase
    i64* part_acc = nullptr;        // batched: a bank's partial piles [K slices][streams][N]
    int* rowinfo = nullptr;        // [B][8]
    i64* wte = nullptr;
    i64* wpe = nullptr;
    // the Pythia machine (kind 1, foundation0/pythia_base2.py): norms with their own gain and offset, the embed
    // table with a power of two per word, the turns' cos / sin, the scores' half-log2(head size)
    int kind = 0;
    int* ng[12][2] = {};  i64* nb[12][2] = {};  int nge[12][2] = {};
    int* fg = nullptr;    i64* fb = nullptr;    int fge = 0;
    short* ew = nullptr;  int* ee = nullptr;
    short* ew2 = nullptr;                               // split digits: the subtracted word table (row = ew - ew2)
    int* cosT = nullptr;  int* sinT = nullptr;  int rot = 0;
    i64 half = 0, ehalf = 0;
    // batch 1: k_gemv's MODE bits (the complement machine, the float gauge and edge, split digits), the float
    // turn and arrival
    int mode = 0;
    bool fturn = false, farr = false;
    // a run's steps after its first take the race of the step before into their first kernel, and the run ends
    // with the race: batch 1 (GPT-2 with every stage integer, the full head read and the plain stream) into layer
    // 0's qkv (PRO_RACE), the batched machines into the word's light or row kernel (PRO_RACE_EMBED,
    // PY_RACE_EMBED)
    bool fold = false;
    // batch 1: steps at positions from att_split on run the attention spread over chunks of positions (-1: never);
    // att_long is the structure of the steps being launched or captured
    int att_split = -1;
    bool att_long = false;
    i64 *asc = nullptr, *acm = nullptr, *aacc = nullptr;   // its score row [12][ctx], chunk maxima, accumulators
    int ncm = 0;
    int* hpin = nullptr;      // pinned host words: the control block and every stream's words of a generate call
    double *cosF = nullptr, *sinF = nullptr;            // turn=float: [npos][rot / 2]
    double* KF = nullptr;                               // arrival=float: [L][12 heads][ctx][64] keys as float64
    // the collapsing top read (batch 1): planes, the first stage's candidates, the light, the step's survivors
    int8_t* top_hi = nullptr;                           // high bytes in the head's column tiles
    uint8_t* top_lo = nullptr;                          // [vocab][768] low bytes, word by word
    int* cand_j = nullptr; i64* cand_h = nullptr; i64* cand_c = nullptr;   // [head_grid][TOP_CAP]
    int* top_x = nullptr; i64* top_f = nullptr;         // [768], [4]
    int* top_n = nullptr; int* top_w = nullptr; i64* top_pile = nullptr; i64* top_score = nullptr;   // [1], [1024] x3
    sm_tables T;
    // state
    i64 *R = nullptr, *QKV = nullptr, *att = nullptr, *hid = nullptr;
    int *att32 = nullptr, *hid32 = nullptr;   // batched: the attention and hidden rows' low 32 bits (k_gemm's SRC)
    i64* R0 = nullptr;                                  // batch 1: the entering row of the next position
    i64* attor = nullptr;                               // [rows][12] OR of |att| over each head's values
    i64* hidor = nullptr;                               // [rows][192] OR of |hid| over each fc tile's columns
    int* sfacts = nullptr;                              // [4][rows][4] mproj's K slices' light facts
    short* K16 = nullptr;                              // [L][B][12 heads][ctx][64] int16 (+32768 as 32767)
    i64* V64 = nullptr;                                // [L][B][12 heads][ctx][64] rows with a value past 32 bits,
                                                       // whole (not with the float arrival)
    int* VW = nullptr;                                 // [L][B][12][ctx] the rows held in V64
    int* vbig = nullptr;                               // [L][B][12] heads holding a value past 32 bits
    i64* KM = nullptr;                                 // [L][B][12][ctx] the +32768 dimensions of each key
    int *EK = nullptr, *V = nullptr;                   // [L][B][12][ctx], [L][B][12 heads][ctx][64]
    int* seq = nullptr;                                 // [B][ctx + 1]
    int* words = nullptr;                               // [B][ctx + 1]
    int* ctl = nullptr;
    i64* part_v = nullptr;
    int* part_i = nullptr;
    // record
    i64 *r_x16 = nullptr, *r_exls = nullptr, *r_pile = nullptr, *r_qkv = nullptr, *r_att = nullptr, *r_hid = nullptr,
        *r_resid = nullptr, *r_hx16 = nullptr, *r_hexls = nullptr, *r_hpile = nullptr, *r_logits = nullptr;
    i64 *r_gauge = nullptr, *r_fcpre = nullptr, *r_hgauge = nullptr;   // Pythia: gauges [L][2][768], fc before the edge
    // captured decode steps: [0] graph_steps whole steps, [1] one whole step, [2] one step's layers, [3] its head,
    // [4], [5]: [0], [1] with the attention spread over chunks of positions; one capture for each position slot a
    // replay starts from (gflip: the replay ends on the other slot)
    hipGraphExec_t gexec[6][2] = {};
    hipGraph_t graph[6][2] = {};
    bool gflip[6] = {};
    int gsteps = 16;
    int par = 0;                   // batched streams: the slot that holds the position of the next step
    // profiling: an event pair around each step's head kernel (the largest single launch)
    // prompt passes: row r of a pass is position pfmap[r] & 0xFFFF of stream pfmap[r] >> 16
    int* pfmap = nullptr;                               // [B][ctx]
    std::vector<int> h_pfmap;
    int h_pfpos = 0;
    // host mirror
    int h_plen = 0, h_pos = 0, h_words = 0, h_recpos = -1;
    std::vector<std::vector<int>> prompts;
};

static bool read_file(const std::string& path, std::vector<char>& out) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) return false;
    std::streamsize n = f.tellg();
    f.seekg(0);
    out.resize((size_t)n);
    return n == 0 || (bool)f.read(out.data(), n);
}

template <typename T>
static int read_array(const std::string& path, std::vector<T>& v, size_t count) {
    std::vector<char> raw;
    if (!read_file(path, raw)) return fail(SM_E_IO, "cannot read " + path);
    if (count != (size_t)-1 && raw.size() != count * sizeof(T))
        return fail(SM_E_IO, path + ": expected " + std::to_string(count * sizeof(T)) + " bytes, found " + std::to_string(raw.size()));
    if (raw.size() % sizeof(T)) return fail(SM_E_IO, path + ": size is not a whole number of elements");
    v.resize(raw.size() / sizeof(T));
    memcpy(v.data(), raw.data(), raw.size());
    return SM_OK;
}

// the few manifest.json facts we need (base2_gpu.py:16): banks[{name, nin, nout}], log2_768, eps40, arrival_len
static bool json_int(const std::string& s, size_t from, const std::string& key, long long& v) {
    size_t k = s.find("\"" + key + "\"", from);
    if (k == std::string::npos) return false;
    size_t c = s.find(':', k);
    if (c == std::string::npos) return false;
    c++;
    while (c < s.size() && (s[c] == ' ' || s[c] == '\t' || s[c] == '\n' || s[c] == '\r')) c++;
    char* end = nullptr;
    v = strtoll(s.c_str() + c, &end, 10);
    return end != s.c_str() + c;
}

struct BankInfo { std::string name; long long nin, nout; };

static int parse_manifest(const std::string& text, std::vector<BankInfo>& banks, long long& log768, long long& eps40, long long& alen) {
    size_t b = text.find("\"banks\"");
    if (b == std::string::npos) return fail(SM_E_IO, "manifest.json: no banks");
    size_t lb = text.find('[', b), rb = text.find(']', b);
    if (lb == std::string::npos || rb == std::string::npos) return fail(SM_E_IO, "manifest.json: malformed banks");
    size_t cur = lb;
    while (true) {
        size_t ob = text.find('{', cur);
        if (ob == std::string::npos || ob > rb) break;
        size_t cb = text.find('}', ob);
        std::string obj = text.substr(ob, cb - ob + 1);
        BankInfo bi;
        size_t nk = obj.find("\"name\"");
        if (nk == std::string::npos) return fail(SM_E_IO, "manifest.json: bank without name");
        size_t q1 = obj.find('"', obj.find(':', nk) + 1), q2 = obj.find('"', q1 + 1);
        bi.name = obj.substr(q1 + 1, q2 - q1 - 1);
        if (!json_int(obj, 0, "nin", bi.nin) || !json_int(obj, 0, "nout", bi.nout)) return fail(SM_E_IO, "manifest.json: bank sizes");
        banks.push_back(bi);
        cur = cb + 1;
    }
    std::string rest = text.substr(0, lb) + text.substr(rb);
    if (!json_int(rest, 0, "log2_768", log768) || !json_int(rest, 0, "eps40", eps40) || !json_int(rest, 0, "arrival_len", alen))
        return fail(SM_E_IO, "manifest.json: constants missing");
    return SM_OK;
}

// "norms": [{"name": "ln1.0", "ge": -14}, ...] (the Pythia layout)
static int parse_norms(const std::string& text, std::vector<std::pair<std::string, long long>>& norms) {
    size_t b = text.find("\"norms\"");
    if (b == std::string::npos) return fail(SM_E_IO, "manifest.json: no norms");
    size_t lb = text.find('[', b), rb = text.find(']', b);
    if (lb == std::string::npos || rb == std::string::npos) return fail(SM_E_IO, "manifest.json: malformed norms");
    for (size_t cur = lb;;) {
        size_t ob = text.find('{', cur);
        if (ob == std::string::npos || ob > rb) break;
        size_t cb = text.find('}', ob);
        std::string obj = text.substr(ob, cb - ob + 1);
        size_t nk = obj.find("\"name\"");
        long long ge;
        if (nk == std::string::npos || !json_int(obj, 0, "ge", ge)) return fail(SM_E_IO, "manifest.json: malformed norm");
        size_t q1 = obj.find('"', obj.find(':', nk) + 1), q2 = obj.find('"', q1 + 1);
        norms.emplace_back(obj.substr(q1 + 1, q2 - q1 - 1), ge);
        cur = cb + 1;
    }
    return SM_OK;
}

static void machine_free(sm_machine* m) {
    if (!m) return;
    for (int i = 0; i < 6; i++)
        for (int j = 0; j < 2; j++) {
            if (m->gexec[i][j]) (void)hipGraphExecDestroy(m->gexec[i][j]);
            if (m->graph[i][j]) (void)hipGraphDestroy(m->graph[i][j]);
        }
    for (int l = 0; l < 12; l++)
        for (int k = 0; k < 4; k++) { free_plate(m->bank[l][k]); free_mfma_plate(m->mbank[l][k]); }
    free_plate(m->head);
    free_mfma_plate(m->mhead);
    tables_free(m->T);
    void* ps[] = {m->pfmap, m->planes, m->part_acc, m->rowinfo, m->wte, m->wpe, m->R, m->R0, m->QKV, m->att, m->att32, m->hid32, m->attor, m->hidor, m->sfacts, m->hid, m->K16, m->KM, m->EK, m->V, m->seq, m->words, m->ctl,
                  m->part_v, m->part_i, m->r_x16, m->r_exls, m->r_pile, m->r_qkv, m->r_att, m->r_hid, m->r_resid,
                  m->r_hx16, m->r_hexls, m->r_hpile, m->r_logits, m->r_gauge, m->r_fcpre, m->r_hgauge,
                  m->fg, m->fb, m->ew, m->ee, m->ew2, m->cosT, m->sinT, m->cosF, m->sinF, m->KF,
                  m->top_hi, m->top_lo, m->cand_j, m->cand_h, m->cand_c, m->top_x, m->top_f, m->top_n, m->top_w,
                  m->top_pile, m->top_score, m->asc, m->acm, m->aacc, m->V64, m->VW, m->vbig};
    for (void* p : ps) hfree(p);
    for (int l = 0; l < 12; l++)
        for (int j = 0; j < 2; j++) { hfree(m->ng[l][j]); hfree(m->nb[l][j]); }
    if (m->hpin) (void)hipHostFree(m->hpin);
    if (m->st) (void)hipStreamDestroy(m->st);
    delete m;
}

// the launch sequence of one decode step (all streams, one position each): the layers and/or the head
enum { STEP_ALL = 3, STEP_LAYERS = 1, STEP_HEAD = 2 };

// the head kernel's blocks: two per CU, each streaming about ntiles / 512 column tiles
static int head_rows_grid(int ntiles) { return std::min(512, ntiles); }

// the many-stream attention over `rows` rows (one block a head and row): 512-thread blocks where the grid has at
// most ATT_WIDE_BLOCKS blocks (more of each block's cache loads in flight), else 256.  Measured (same box,
// identical words): Pythia at 32 streams 62.5 k against 62.0 k tokens/s with 512; GPT-2 at 64 streams 108.5 k
// against 113.7 k (768 blocks of 512 threads no longer fit three waves a SIMD beside the rest)
#ifndef ATT_WIDE_BLOCKS
#define ATT_WIDE_BLOCKS 384
#endif
template <int MODEL>
static void attend_rows(sm_machine* m, int rows, const AttArgs& a) {
    // (the arrivals read from the table: from their formula the 64-stream step measured 0.6 % slower)
    if (12 * rows <= ATT_WIDE_BLOCKS)
        launch(m->cfg.profile, "attend", k_attend<MODEL, 0, 1, 0, 512>, dim3(12, rows), dim3(512), (size_t)m->ctx * 12, m->st, a);
    else
        launch(m->cfg.profile, "attend", k_attend<MODEL, 0, 1>, dim3(12, rows), dim3(NTHR), (size_t)m->ctx * 12, m->st, a);
}

// batched streams: every bank is [light kernel (one block per stream) -> MFMA kernel (one block per 16 columns)]
//
// rowmap != null: a pass of nrows prompt rows (row r: position rowmap[r] & 0xFFFF of stream rowmap[r] >> 16)
// instead of one position of every stream.  Their words are known, so no head runs, and the last layer only
// stores keys and values (its attention and banks feed the head alone); nothing is recorded.
// fused: the race of the step before runs in the word's light (PRO_RACE_EMBED), which reads that step's position
// slot and writes the other one, read by every later kernel of this step; race: the step ends with k_race_rows
template <int RT>
static int launch_step_batched(sm_machine* m, int parts, int nrows = 0,
                               const int* rowmap = nullptr, bool fused = false, bool race = true) {
    const Tables tb = m->T.tb();
    int* ctl = m->ctl;
    const bool fold = m->fold && fused && !rowmap && parts == STEP_ALL;
    if (!m->fold || rowmap || parts != STEP_ALL) race = true;
    int* const posA = ctl + (m->par ? CTL_POS1 : CTL_POS);
    int* const posp = fold ? ctl + (m->par ? CTL_POS : CTL_POS1) : posA;
    if (fold) m->par ^= 1;
    const int B = rowmap ? nrows : m->B;
    const int* recp = rowmap ? nullptr : ctl + CTL_RECPOS;
    auto light_args = [&](int K, const i64* X, i64* rx16, i64* rexls) {
        LightArgs a{};
        a.K = K; a.rows = B; a.X = X; a.wte = m->wte; a.wpe = m->wpe; a.seq = m->seq; a.seq_stride = m->ctx + 1;
        a.Rw = m->R; a.pos = posp; a.plen = ctl + CTL_PLEN;
        a.planes = m->planes; a.rowinfo = m->rowinfo; a.tb = tb;
        a.rec_pos = recp; a.rx16 = rx16; a.rexls = rexls; a.rowmap = rowmap;
        return a;
    };
    // mproj's epilogue (from its four K slices of partial piles) added into the stream, then the next light
    auto finish_light = [&](const MfmaPlate& P, i64* rpile, i64* rout, i64* rx16, i64* rexls, int ls_row) {
        LightArgs a = light_args(P.N, nullptr, rx16, rexls);
        a.ls_row = ls_row;
        a.part = m->part_acc; a.kin = P.K; a.csum = P.csum; a.we = P.e; a.bias = P.b; a.Y = m->R;
        a.rpile_in = rpile; a.rout_in = rout; a.sfacts = m->sfacts;
        launch(m->cfg.profile, "light.add_gauge", k_light<768, PRO_ADD_GAUGE, 192, 4>, dim3(B), dim3(192), 0, m->st, a);
    };
    auto gemm_args = [&](const MfmaPlate& P, i64* Y, int ystride, i64* rpile, i64* rout) {
        GemmArgs a{};
        a.K = P.K; a.N = P.N; a.rows = B; a.RT = RT; a.W = P.W; a.csum = P.csum; a.we = P.e; a.bias = P.b;
        a.planes = m->planes; a.rowinfo = m->rowinfo; a.Y = Y; a.ystride = ystride; a.tb = tb;
        a.pos = posp; a.plen = ctl + CTL_PLEN; a.rec_pos = recp; a.rpile = rpile; a.rout = rout;
        a.part = m->part_acc;
        return a;
    };
    for (int l = 0; l < 12 && (parts & STEP_LAYERS); l++) {
        i64* rx = m->r_x16 + (size_t)l * 4 * 3072;
        i64* re = m->r_exls + (size_t)l * 4 * 2;
        i64* rp = m->r_pile + (size_t)l * 4 * 3072;
        if (l == 0) {      // the word enters; later layers get their light from the previous layer's last kernel
            LightArgs a = light_args(768, m->R, rx, re);
            if (fold) {    // the race of the step before, then the word it feeds back
                a.pos = posA; a.pos_next = posp; a.nwords = ctl + CTL_NWORDS;
                a.part_v = m->part_v; a.part_i = m->part_i; a.nblk = head_rows_grid(m->mhead.ntiles);
                a.words = m->words; a.words_stride = m->ctx + 1; a.seqw = m->seq;
                launch(m->cfg.profile, "light.embed.race", k_light<768, PRO_RACE_EMBED, 192, 1>, dim3(B), dim3(192), 0, m->st, a);
            } else {
                launch(m->cfg.profile, "light.embed", k_light<768, PRO_EMBED, 192, 1>, dim3(B), dim3(192), 0, m->st, a);
            }
        }
        {
            GemmArgs a = gemm_args(m->mbank[l][0], m->QKV, 2304, rp, m->r_qkv + l * 2304);
            launch(m->cfg.profile, "qkv", k_gemm<768, 1, 1, EPI_GAUGED>, dim3(m->mbank[l][0].ntiles, RT), dim3(256), 0, m->st, a);
        }
        {
            AttArgs a{};
            const size_t per = (size_t)m->B * m->ctx;
            a.QKV = m->QKV; a.K16 = m->K16 + l * per * 768; a.KM = m->KM + l * per * 12; a.EK = m->EK + l * per * 12; a.V = m->V + l * per * 768;
            a.V64 = m->V64 ? m->V64 + l * per * 768 : nullptr; a.VW = m->VW ? m->VW + l * per * 12 : nullptr;
            a.vbig = m->vbig ? m->vbig + (size_t)l * m->B * 12 : nullptr;
            a.out = m->att; a.pos = posp; a.ctx = m->ctx; a.tb = tb; a.err = ctl + CTL_ERR;
            a.rec_pos = recp; a.ratt = m->r_att + l * 768; a.rowmap = rowmap; a.out_or = m->attor; a.out32 = m->att32;
            if (rowmap) {
                launch(m->cfg.profile, "kv_rows", k_kv_rows<0>, dim3(12, B), dim3(128), 0, m->st, a);
                if (l == 11) break;
                attend_rows<0>(m, B, a);
            } else {
                attend_rows<0>(m, m->B, a);
            }
        }
        {   // proj: the attention rows' light formed in the bank, the plain bank added into the stream; then the
            // stream's light and gauge for fc (a light formed in fc's own blocks measured slower: the gauge's
            // table reads would follow the row's conversion there)
            GemmArgs a = gemm_args(m->mbank[l][1], m->R, 768, rp + 3072, m->r_resid + (l * 2 + 0) * 768);
            a.X = m->att; a.X32 = m->att32; a.xstride = 768; a.orw = m->attor; a.rx16 = rx + 3072; a.rexls = re + 2;
            launch(m->cfg.profile, "proj", k_gemm<768, 1, 1, EPI_PLAIN_ADD, 12>, dim3(m->mbank[l][1].ntiles, RT), dim3(256), 0, m->st, a);
            LightArgs g = light_args(768, m->R, rx + 2 * 3072, re + 4);
            launch(m->cfg.profile, "light.gauge", k_light<768, PRO_GAUGE, 192, 1>, dim3(B), dim3(192), 0, m->st, g);
        }
        {   // fc: gauged, the edge, written (the hidden rows) with their OR words
            GemmArgs a = gemm_args(m->mbank[l][2], m->hid, 3072, rp + 2 * 3072, m->r_hid + l * 3072);
            a.orw_out = m->hidor; a.Y32 = m->hid32;
            launch(m->cfg.profile, "fc", k_gemm<768, 1, 1, EPI_GAUGED_EDGE>, dim3(m->mbank[l][2].ntiles, RT), dim3(256), 0, m->st, a);
        }
        {   // mproj: the hidden rows' light formed in each K slice's blocks; partial piles and slice facts
            GemmArgs a = gemm_args(m->mbank[l][3], nullptr, 0, nullptr, nullptr);
            a.X = m->hid; a.X32 = m->hid32; a.xstride = 3072; a.orw = m->hidor; a.rx16 = rx + 3 * 3072; a.rexls = re + 6;
            a.sfacts = m->sfacts;
            launch(m->cfg.profile, "mproj.part", k_gemm<3072, 3, 4, EPI_PART, 192>, dim3(m->mbank[l][3].ntiles / 3 * 4, RT), dim3(256), 0, m->st, a);
        }
        const bool last = l == 11;     // the last stream update lights the head
        finish_light(m->mbank[l][3], rp + 3 * 3072, m->r_resid + (l * 2 + 1) * 768,
                     last ? m->r_hx16 : m->r_x16 + (size_t)(l + 1) * 4 * 3072, last ? m->r_hexls : m->r_exls + (size_t)(l + 1) * 4 * 2,
                     last && !rowmap);     // the head takes LS and the power factor made here
    }
    if ((parts & STEP_HEAD) && !rowmap) {
        GemmArgs a = gemm_args(m->mhead, nullptr, 0, m->r_hpile, nullptr);
        // the head: each wave's row tile of lights in registers, weight tiles streamed through LDS
        const int grid = head_rows_grid(m->mhead.ntiles), parts = grid;
        a.part_v = m->part_v; a.part_i = m->part_i; a.nblk = parts; a.rlogits = m->r_logits;
        launch(m->cfg.profile, "head", k_head_rows<RT, EPI_HEAD>, dim3(grid), dim3(256), 0, m->st, a);
        RaceArgs r{};
        r.part_v = m->part_v; r.part_i = m->part_i; r.nblk = parts; r.seq = m->seq; r.seq_stride = m->ctx + 1;
        r.words = m->words; r.words_stride = m->ctx + 1; r.pos = posp; r.plen = ctl + CTL_PLEN;
        r.pos_next = ctl + (m->par ? CTL_POS : CTL_POS1); r.nwords = ctl + CTL_NWORDS;
        if (race) {
            launch(m->cfg.profile, "race", k_race_rows, dim3(B), dim3(256), 0, m->st, r);
            m->par ^= 1;                             // the next step reads the slot this race writes
        }
    }
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// the batch-1 head: tiles of 4 columns, four waves per block, two blocks per CU by default (measured on the
// 768 x 50257 plate: 4-column tiles at 512 blocks 15.7 us; 8-column tiles at 256 blocks 17.3 us (one wave a
// SIMD, 256 VGPRs), at 512 blocks 19.2 us; 2-column tiles at 768 blocks 16.2 us)
#define HEAD_WPB 4
#define HEAD_TC 4
#define TOP_RECORD 1024       // survivors of the top read's last step kept for sm_read

// batch 1: the race over the head blocks' bests, the word fed back, the next position's entering row (k_race1);
// k_embed1 writes the entering row of the current position (the first step of a run)
static Race1Args race1_args(sm_machine* m) {
    int* ctl = m->ctl;
    Race1Args r{};
    r.part_v = m->part_v; r.part_i = m->part_i; r.nblk = m->head_grid;
    r.seq = m->seq; r.words = m->words; r.pos = ctl + (m->par ? CTL_POS1 : CTL_POS); r.plen = ctl + CTL_PLEN;
    r.nwords = ctl + CTL_NWORDS;
    r.R0 = m->R0;
    r.npos = m->kind == 1 ? m->ctx : m->npos;
    r.wte = m->wte; r.wpe = m->wpe; r.ew = m->ew; r.ee = m->ee; r.ew2 = m->ew2;
    return r;
}
static void launch_race1(sm_machine* m) {
    if (m->kind == 1) launch(m->cfg.profile, "race", k_race1<1>, dim3(1), dim3(256), 0, m->st, race1_args(m));
    else if (m->cfg.inv) launch(m->cfg.profile, "race", k_race1<0, 1>, dim3(1), dim3(256), 0, m->st, race1_args(m));
    else launch(m->cfg.profile, "race", k_race1<0>, dim3(1), dim3(256), 0, m->st, race1_args(m));
}
static void launch_embed1(sm_machine* m) {
    if (m->kind == 1) launch(m->cfg.profile, "embed", k_embed1<1>, dim3(1), dim3(256), 0, m->st, race1_args(m));
    else if (m->cfg.inv) launch(m->cfg.profile, "embed", k_embed1<0, 1>, dim3(1), dim3(256), 0, m->st, race1_args(m));
    else launch(m->cfg.profile, "embed", k_embed1<0>, dim3(1), dim3(256), 0, m->st, race1_args(m));
}

// the next GEMV phase's plate for this phase's blocks to request early (GemvArgs::pf): its first wpb tiles
// of every block of its grid
static void set_pf(GemvArgs& a, const DevPlate& next, int wpb, int grid) {
    a.pf = reinterpret_cast<const char*>(next.W);
    a.pf_lines = wpb * next.tc * next.nin * 2 / 128;
    a.pf_nblk = grid;
    a.pf_total = (int)((size_t)next.ntiles * next.tc * next.nin * 2 / 128);
}
static int grid4(const DevPlate& P) { return (P.ntiles + 3) / 4; }   // four waves a block, a tile a wave
static int grid2(const DevPlate& P) { return (P.ntiles + 1) / 2; }   // two waves a block
// the head's first stage for the next phase to pull: the full table's tiles, or the top read's high bytes
static void set_pf_head(sm_machine* m, GemvArgs& a) {
    if (m->cfg.top_read) {
        a.pf = reinterpret_cast<const char*>(m->top_hi);
        a.pf_lines = HEAD_WPB * HEAD_TC * 768 / 128;
        a.pf_nblk = m->head_grid;
        a.pf_total = (int)((size_t)m->head.ntiles * HEAD_TC * 768 / 128);
    } else {
        set_pf(a, m->head, HEAD_WPB, m->head_grid);
    }
}

// a batch-1 GEMV phase: rec selects the instantiation that records (launched only for the recorded step), the
// machine's MODE bits the rest (only those the phase has; the complement machine is never mixed with float stages)
static constexpr int phase_modes(int PRO, int EPI) {
    return (PRO == PRO_GAUGE || PRO == PRO_TO16 || PRO == PRO_ATT ? MODE_INV : 0) |
           (PRO == PRO_GAUGE || PRO == PRO_PGAUGE ? MODE_FGAUGE : 0) |
           (EPI == EPI_GAUGED_EDGE || EPI == EPI_PLAIN_EDGE ? MODE_FEDGE : 0) |
           ((PRO == PRO_PGAUGE || PRO == PRO_TO16 || PRO == PRO_PATT) &&
                    (EPI == EPI_PLAIN || EPI == EPI_PLAIN_EDGE || EPI == EPI_PHEAD || EPI == EPI_PLAIN_ADD) ? MODE_SPLIT : 0);
}
template <int NIN, int TC, int WPB, int PRO, int EPI, int M = 0>
static void gemv_mode(sm_machine* m, int mode, bool rec, const char* name, int grid, const GemvArgs& a) {
    if constexpr (M < 16) {
        if constexpr ((M & ~phase_modes(PRO, EPI)) == 0 && (M == MODE_INV || !(M & MODE_INV))) {
            if (mode == M) {
                if (rec) launch(m->cfg.profile, name, k_gemv<NIN, TC, WPB, PRO, EPI, 1, M>, dim3(grid), dim3(64 * WPB), 0, m->st, a);
                else launch(m->cfg.profile, name, k_gemv<NIN, TC, WPB, PRO, EPI, 0, M>, dim3(grid), dim3(64 * WPB), 0, m->st, a);
                return;
            }
        }
        gemv_mode<NIN, TC, WPB, PRO, EPI, M + 1>(m, mode, rec, name, grid, a);
    }
}
template <int NIN, int TC, int WPB, int PRO, int EPI>
static void gemv(sm_machine* m, bool rec, const char* name, int grid, const GemvArgs& a) {
    gemv_mode<NIN, TC, WPB, PRO, EPI>(m, m->mode & phase_modes(PRO, EPI), rec, name, grid, a);
}
// batch-1 attention: the integer arrival (turn=float: its FTURN instantiation), or arrival=float
template <int MODEL, int FTURN>
static void attend1_t(sm_machine* m, bool rec, AttArgs a) {
    if constexpr (!FTURN) {
        if (m->att_long) {                    // the attention spread over chunks of positions (sm_attend_split.hip)
            // two launches: the divisor and the output row are formed by proj's blocks from the accumulators
            // (PRO_ATT / PRO_PATT), in place of k_att_finish
            a.asc = m->asc; a.acm = m->acm; a.aacc = m->aacc; a.ncm = m->ncm;
            const dim3 grid(12, m->ncm);
            launch(m->cfg.profile, "attend.scores", k_att_scores<MODEL>, grid, dim3(256), 0, m->st, a);
            if (m->T.verified) launch(m->cfg.profile, "attend.mix", k_att_mix<MODEL, 1>, grid, dim3(256), 0, m->st, a);
            else launch(m->cfg.profile, "attend.mix", k_att_mix<MODEL, 0>, grid, dim3(256), 0, m->st, a);
            return;
        }
    }
    if (m->farr) {
        if (rec) launch(m->cfg.profile, "attend", k_attend_f<MODEL, FTURN, 1>, dim3(12), dim3(256), (size_t)m->ctx * 8, m->st, a);
        else launch(m->cfg.profile, "attend", k_attend_f<MODEL, FTURN, 0>, dim3(12), dim3(256), (size_t)m->ctx * 8, m->st, a);
        return;
    }
    // the arrivals from their formula where the tables are the reference's (the create-time check)
    const size_t sh = (size_t)m->ctx * 12;
    if (m->T.verified) {
        if (rec) launch(m->cfg.profile, "attend", k_attend<MODEL, 1, 1, FTURN, NTHR, 1>, dim3(12, 1), dim3(NTHR), sh, m->st, a);
        else launch(m->cfg.profile, "attend", k_attend<MODEL, 1, 0, FTURN, NTHR, 1>, dim3(12, 1), dim3(NTHR), sh, m->st, a);
    } else {
        if (rec) launch(m->cfg.profile, "attend", k_attend<MODEL, 1, 1, FTURN>, dim3(12, 1), dim3(NTHR), sh, m->st, a);
        else launch(m->cfg.profile, "attend", k_attend<MODEL, 1, 0, FTURN>, dim3(12, 1), dim3(NTHR), sh, m->st, a);
    }
}
template <int MODEL>
static void attend1(sm_machine* m, bool rec, AttArgs a, int layer) {
    a.cosF = m->cosF; a.sinF = m->sinF;
    a.KF = m->KF ? m->KF + (size_t)layer * 12 * m->ctx * 64 : nullptr;
    if constexpr (MODEL == 1) {
        if (m->fturn) { attend1_t<1, 1>(m, rec, a); return; }
    }
    attend1_t<MODEL, 0>(m, rec, a);
}

// The Pythia machine at batch 1 (foundation0/pythia_base2.py:153-160), five phases a layer.  Both gauges read
// the stream before either half adds to it (the parallel residual R + At + Mo, :155-157): qkv and fc first.
static int launch_step_pythia(sm_machine* m, int parts, bool rec) {
    const Tables tb = m->T.tb();
    int* ctl = m->ctl;
    for (int l = 0; l < 12 && (parts & STEP_LAYERS); l++) {
        GemvArgs base{};
        base.tb = tb;
        base.pos = ctl + CTL_POS;
        base.rec_pos = ctl + CTL_RECPOS;
        base.err = ctl + CTL_ERR;                      // the reference's rshift assert (pythia_base2.py:63)
        auto plate = [&](GemvArgs& a, const DevPlate& P, int k) {
            a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
            a.W2 = reinterpret_cast<const int4*>(P.W2);
            a.rx16 = m->r_x16 + (l * 4 + k) * 3072; a.rexls = m->r_exls + (l * 4 + k) * 2;
            a.rpile = m->r_pile + (l * 4 + k) * 3072;
        };
        const i64* Rin = l == 0 ? m->R0 : m->R;        // layer 0 reads the entering row (k_race1 / k_embed1)
        // qkv: gauge ln1 of R, plain (:113, 130)
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][0];
            plate(a, P, 0);
            a.X = Rin; a.Y = m->QKV; a.rout = m->r_qkv + l * 2304; a.rg = m->r_gauge + (l * 2 + 0) * 768;
            a.ng = m->ng[l][0]; a.nb = m->nb[l][0]; a.nge = m->nge[l][0];
            set_pf(a, m->bank[l][2], 4, grid4(m->bank[l][2]));
            gemv<768, 2, 4, PRO_PGAUGE, EPI_PLAIN>(m, rec, "qkv", (P.ntiles + 3) / 4, a);
        }
        // fc: gauge ln2 of the same R, plain, edge (:156)
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][2];
            plate(a, P, 2);
            a.X = Rin; a.Y = m->hid; a.rout = m->r_fcpre + l * 3072; a.rout2 = m->r_hid + l * 3072;
            a.rg = m->r_gauge + (l * 2 + 1) * 768;
            a.ng = m->ng[l][1]; a.nb = m->nb[l][1]; a.nge = m->nge[l][1];
            set_pf(a, m->bank[l][1], 2, grid2(m->bank[l][1]));
            gemv<768, 2, 4, PRO_PGAUGE, EPI_PLAIN_EDGE>(m, rec, "fc", (P.ntiles + 3) / 4, a);
        }
        // attention with turns (:125-141)
        {
            AttArgs a{};
            const size_t per = (size_t)m->B * m->ctx;
            a.QKV = m->QKV; a.K16 = m->K16 + l * per * 768; a.KM = m->KM + l * per * 12; a.EK = m->EK + l * per * 12; a.V = m->V + l * per * 768;
            a.V64 = m->V64 ? m->V64 + l * per * 768 : nullptr; a.VW = m->VW ? m->VW + l * per * 12 : nullptr;
            a.vbig = m->vbig ? m->vbig + (size_t)l * m->B * 12 : nullptr;
            a.out = m->att; a.pos = ctl + CTL_POS; a.ctx = m->ctx; a.tb = tb; a.err = ctl + CTL_ERR;
            a.rec_pos = ctl + CTL_RECPOS; a.ratt = m->r_att + l * 768;
            a.cosT = m->cosT; a.sinT = m->sinT; a.rot = m->rot; a.half = m->half; a.ehalf = m->ehalf;
            // proj: plain of the attention row, added to R (At; layer 0: to the entering row)
            GemvArgs g = base;
            const DevPlate& P = m->bank[l][1];
            plate(g, P, 1);
            g.X = m->att; g.Y = m->R; g.Yb = Rin; g.rout = m->r_resid + (l * 2 + 0) * 768;
            set_pf(g, m->bank[l][3], 4, grid4(m->bank[l][3]));
            attend1<1>(m, rec, a, l);
            if (m->att_long) {          // the attention's output row formed in proj's blocks
                g.aacc = m->aacc; g.ratt = m->r_att + l * 768;
                gemv<768, 2, 2, PRO_PATT, EPI_PLAIN_ADD>(m, rec, "proj", (P.ntiles + 1) / 2, g);
            } else {
                gemv<768, 2, 2, PRO_TO16, EPI_PLAIN_ADD>(m, rec, "proj", (P.ntiles + 1) / 2, g);
            }
        }
        // mproj: plain of the edge row, added to R (Mo)
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][3];
            plate(a, P, 3);
            a.X = m->hid; a.Y = m->R; a.Yb = m->R; a.rout = m->r_resid + (l * 2 + 1) * 768;
            if (l < 11) set_pf(a, m->bank[l + 1][0], 4, grid4(m->bank[l + 1][0]));
            else set_pf(a, m->head, HEAD_WPB, m->head_grid);
            gemv<3072, 1, 4, PRO_TO16, EPI_PLAIN_ADD>(m, rec, "mproj", (P.ntiles + 3) / 4, a);
        }
    }
    // head: gauge lnf, plain with no bias, race (:158-160)
    if (parts & STEP_HEAD) {
        GemvArgs a{};
        a.tb = tb;
        a.err = ctl + CTL_ERR;
        a.pos = ctl + CTL_POS; a.rec_pos = ctl + CTL_RECPOS;
        const DevPlate& P = m->head;
        a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
        a.W2 = reinterpret_cast<const int4*>(P.W2);
        a.X = m->R;
        a.ng = m->fg; a.nb = m->fb; a.nge = m->fge; a.rg = m->r_hgauge;
        a.rx16 = m->r_hx16; a.rexls = m->r_hexls; a.rpile = m->r_hpile; a.rlogits = m->r_logits;
        a.part_v = m->part_v; a.part_i = m->part_i;
        gemv<768, HEAD_TC, HEAD_WPB, PRO_PGAUGE, EPI_PHEAD>(m, rec, "head", m->head_grid, a);
        launch_race1(m);
    }
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// The Pythia machine, batched.  Light sets: A (ln1 -> qkv) and B (ln2 -> fc), both made by the row kernel; mproj
// and proj light their own rows (fc's hidden rows, the attention rows) in their banks.  A decode step runs four
// launches a layer: [fc | qkv] (one launch), [attention | mproj's K-slice partials] (one launch), proj (R + At +
// Mo: its bank also finishes mproj's partials), the row kernel (the next layer's two gauges, or the head's).  The
// halves of the parallel residual (foundation0/pythia_base2.py:155-157) are independent until proj's epilogue
// adds them, so each paired launch holds one kernel of each.
// rowmap != null: a pass of nrows prompt rows, as in launch_step_batched, one kernel a launch.
template <int RT>
static int launch_step_pythia_batched(sm_machine* m, int parts, int nrows = 0,
                                      const int* rowmap = nullptr, bool fused = false, bool race = true) {
    const Tables tb = m->T.tb();
    int* ctl = m->ctl;
    // (fused, race: as launch_step_batched; the race of the step before runs in the word's row kernel)
    const bool fold = m->fold && fused && !rowmap && parts == STEP_ALL;
    if (!m->fold || rowmap || parts != STEP_ALL) race = true;
    int* const posA = ctl + (m->par ? CTL_POS1 : CTL_POS);
    int* const posp = fold ? ctl + (m->par ? CTL_POS : CTL_POS1) : posA;
    if (fold) m->par ^= 1;
    const int B = rowmap ? nrows : m->B;
    const int* recp = rowmap ? nullptr : ctl + CTL_RECPOS;
    const size_t PL = (size_t)4 * 48 * 3 * 1024, RC = m->RC;
    signed char* pA = m->planes; signed char* pB = m->planes + PL;      // the two gauges' lights (qkv, fc)
    int* rA = m->rowinfo; int* rB = m->rowinfo + RC * 8;
    i64* P0 = m->part_acc;                          // mproj's partial piles
    auto gemm_args = [&](const MfmaPlate& P, signed char* planes, int* rowinfo) {
        GemmArgs a{};
        a.K = P.K; a.N = P.N; a.rows = B; a.RT = RT; a.W = P.W; a.csum = P.csum; a.we = P.e; a.bias = P.b;
        a.planes = planes; a.rowinfo = rowinfo; a.tb = tb;
        a.pos = posp; a.plen = ctl + CTL_PLEN; a.rec_pos = recp;
        a.err = ctl + CTL_ERR;                         // the reference's rshift assert (pythia_base2.py:63)
        return a;
    };
    auto rows_args = [&]() {
        PyRowArgs a{};
        a.err = ctl + CTL_ERR;
        a.rows = B; a.R = m->R; a.ew = m->ew; a.ee = m->ee; a.seq = m->seq; a.seq_stride = m->ctx + 1; a.pos = posp;
        a.tb = tb; a.rec_pos = recp; a.rowmap = rowmap;
        return a;
    };
    auto gauges = [&](PyRowArgs& a, int l) {       // the two gauges of layer l (l == 12: lnf for the head)
        a.planes1 = pA; a.rowinfo1 = rA; a.planes2 = pB; a.rowinfo2 = rB;
        if (l < 12) {
            a.ng1 = m->ng[l][0]; a.nb1 = m->nb[l][0]; a.nge1 = m->nge[l][0];
            a.ng2 = m->ng[l][1]; a.nb2 = m->nb[l][1]; a.nge2 = m->nge[l][1];
            a.rg1 = m->r_gauge + (l * 2 + 0) * 768; a.rx1 = m->r_x16 + (l * 4 + 0) * 3072; a.rex1 = m->r_exls + (l * 4 + 0) * 2;
            a.rg2 = m->r_gauge + (l * 2 + 1) * 768; a.rx2 = m->r_x16 + (l * 4 + 2) * 3072; a.rex2 = m->r_exls + (l * 4 + 2) * 2;
        } else {
            a.ng1 = m->fg; a.nb1 = m->fb; a.nge1 = m->fge; a.ng2 = nullptr;
            a.rg1 = m->r_hgauge; a.rx1 = m->r_hx16; a.rex1 = m->r_hexls;
        }
    };
    for (int l = 0; l < 12 && (parts & STEP_LAYERS); l++) {
        i64* rp = m->r_pile + (size_t)l * 4 * 3072;
        if (l == 0) {
            PyRowArgs a = rows_args();
            gauges(a, 0);
            if (fold) {    // the race of the step before, then the word it feeds back
                a.pos = posA; a.pos_next = posp; a.nwords = ctl + CTL_NWORDS; a.plen = ctl + CTL_PLEN;
                a.part_v = m->part_v; a.part_i = m->part_i; a.nblk = head_rows_grid(m->mhead.ntiles);
                a.words = m->words; a.words_stride = m->ctx + 1; a.seqw = m->seq;
                launch(m->cfg.profile, "rows.embed.race", k_py_rows<PY_RACE_EMBED>, dim3(B), dim3(192), 0, m->st, a);
            } else {
                launch(m->cfg.profile, "rows.embed", k_py_rows<PY_EMBED>, dim3(B), dim3(192), 0, m->st, a);
            }
        }
        GemmArgs aq = gemm_args(m->mbank[l][0], pA, rA);              // qkv: plain, written
        aq.Y = m->QKV; aq.ystride = 2304; aq.rpile = rp; aq.rout = m->r_qkv + l * 2304;
        GemmArgs af = gemm_args(m->mbank[l][2], pB, rB);              // fc: plain and edged, with OR words
        af.Y = m->hid; af.ystride = 3072;
        af.rpile = rp + 2 * 3072; af.rout = m->r_fcpre + l * 3072; af.rout2 = m->r_hid + l * 3072;
        af.orw_out = m->hidor; af.Y32 = m->hid32;
        GemmArgs am = gemm_args(m->mbank[l][3], nullptr, nullptr);   // mproj: K-slice partials
        am.part = P0;
        am.X = m->hid; am.X32 = m->hid32; am.xstride = 3072; am.orw = m->hidor; am.sfacts = m->sfacts;
        am.rx16 = m->r_x16 + (l * 4 + 3) * 3072; am.rexls = m->r_exls + (l * 4 + 3) * 2;
        AttArgs at{};                                                  // attention with turns
        {
            const size_t per = (size_t)m->B * m->ctx;
            at.QKV = m->QKV; at.K16 = m->K16 + l * per * 768; at.KM = m->KM + l * per * 12; at.EK = m->EK + l * per * 12;
            at.V = m->V + l * per * 768;
            at.V64 = m->V64 ? m->V64 + l * per * 768 : nullptr; at.VW = m->VW ? m->VW + l * per * 12 : nullptr;
            at.vbig = m->vbig ? m->vbig + (size_t)l * m->B * 12 : nullptr;
            at.out = m->att; at.pos = posp; at.ctx = m->ctx; at.tb = tb; at.err = ctl + CTL_ERR;
            at.rec_pos = recp; at.ratt = m->r_att + l * 768; at.rowmap = rowmap;
            at.cosT = m->cosT; at.sinT = m->sinT; at.rot = m->rot; at.half = m->half; at.ehalf = m->ehalf;
            at.out_or = m->attor; at.out32 = m->att32;
        }
        const int gq = m->mbank[l][0].ntiles, gf = m->mbank[l][2].ntiles, gm = m->mbank[l][3].ntiles / 3 * 4;
        if (!rowmap) {
            // a decode step: the two halves of the layer share launches (fc with qkv, then mproj's partials with
            // the attention), four launches a layer with proj and the row kernel
            launch(m->cfg.profile, "fc+qkv", k_gemm_pair<EPI_PLAIN_EDGE, EPI_PLAIN>, dim3(gf * RT + gq * RT), dim3(256), 0,
                   m->st, af, aq, gf * RT, gf, gq);
            if (m->T.verified)
                launch(m->cfg.profile, "attend+mproj.part", k_attend_mproj<1, 1>, dim3(12 * B + gm * RT), dim3(256),
                       (size_t)m->ctx * 12, m->st, at, am, 12 * B, gm);
            else
                launch(m->cfg.profile, "attend+mproj.part", k_attend_mproj<1, 0>, dim3(12 * B + gm * RT), dim3(256),
                       (size_t)m->ctx * 12, m->st, at, am, 12 * B, gm);
        } else {
            launch(m->cfg.profile, "qkv", k_gemm<768, 1, 1, EPI_PLAIN>, dim3(gq, RT), dim3(256), 0, m->st, aq);
        }
        if (rowmap && l == 11) {   // prompt rows: the last layer only stores its keys and values
            AttArgs a{};
            const size_t per = (size_t)m->B * m->ctx;
            a.QKV = m->QKV; a.K16 = m->K16 + l * per * 768; a.KM = m->KM + l * per * 12; a.EK = m->EK + l * per * 12; a.V = m->V + l * per * 768;
            a.V64 = m->V64 ? m->V64 + l * per * 768 : nullptr; a.VW = m->VW ? m->VW + l * per * 12 : nullptr;
            a.vbig = m->vbig ? m->vbig + (size_t)l * m->B * 12 : nullptr;
            a.ctx = m->ctx; a.tb = tb; a.err = ctl + CTL_ERR; a.rowmap = rowmap;
            a.cosT = m->cosT; a.sinT = m->sinT; a.rot = m->rot; a.half = m->half; a.ehalf = m->ehalf;
            launch(m->cfg.profile, "kv_rows", k_kv_rows<1>, dim3(12, B), dim3(128), 0, m->st, a);
            break;
        }
        if (rowmap) {      // a prompt pass: position by position through each kernel
            launch(m->cfg.profile, "fc", k_gemm<768, 1, 1, EPI_PLAIN_EDGE>, dim3(gf, RT), dim3(256), 0, m->st, af);
            launch(m->cfg.profile, "mproj.part", k_gemm<3072, 3, 4, EPI_PART, 192>, dim3(gm, RT), dim3(256), 0, m->st, am);
            launch(m->cfg.profile, "kv_rows", k_kv_rows<1>, dim3(12, B), dim3(128), 0, m->st, at);
            attend_rows<1>(m, B, at);
        }
        {   // proj: the attention rows' light formed in its bank, added into the stream (R + At)
            GemmArgs g = gemm_args(m->mbank[l][1], nullptr, nullptr);
            g.Y = m->R; g.ystride = 768; g.rpile = rp + 3072; g.rout = m->r_resid + (l * 2 + 0) * 768;
            g.X = m->att; g.X32 = m->att32; g.xstride = 768; g.orw = m->attor;
            g.rx16 = m->r_x16 + (l * 4 + 1) * 3072; g.rexls = m->r_exls + (l * 4 + 1) * 2;
            const MfmaPlate& Pm = m->mbank[l][3];
            if (!rowmap) {     // a decode step: proj's bank also finishes mproj's partials and adds both halves
                g.part2 = P0; g.sfacts2 = m->sfacts; g.csum2 = Pm.csum; g.we2 = Pm.e; g.bias2 = Pm.b; g.kin2 = 3072;
                g.rpile2 = rp + 3 * 3072; g.rout2b = m->r_resid + (l * 2 + 1) * 768;
                launch(m->cfg.profile, "proj", k_gemm<768, 1, 1, EPI_PLAIN_ADD2, 12>, dim3(m->mbank[l][1].ntiles, RT),
                       dim3(256), 0, m->st, g);
            } else {
                launch(m->cfg.profile, "proj", k_gemm<768, 1, 1, EPI_PLAIN_ADD, 12>, dim3(m->mbank[l][1].ntiles, RT),
                       dim3(256), 0, m->st, g);
            }
        }
        {   // (a prompt pass: R += Mo, the parallel residual's other half,) then the next gauges' lights
            PyRowArgs a = rows_args();
            const MfmaPlate& Pm = m->mbank[l][3];
            gauges(a, l + 1);
            if (!rowmap) {
                launch(m->cfg.profile, "rows.gauge", k_py_rows<PY_GAUGE>, dim3(B), dim3(192), 0, m->st, a);
            } else {
                a.partM = P0; a.kinM = 3072; a.sfactsM = m->sfacts; a.csumM = Pm.csum; a.weM = Pm.e; a.biasM = Pm.b;
                a.rpileM = rp + 3 * 3072; a.routM = m->r_resid + (l * 2 + 1) * 768;
                launch(m->cfg.profile, "rows.add", k_py_rows<PY_ADD>, dim3(B), dim3(192), 0, m->st, a);
            }
        }
    }
    if ((parts & STEP_HEAD) && !rowmap) {
        GemmArgs a = gemm_args(m->mhead, pA, rA);
        a.rpile = m->r_hpile;
        const int grid = head_rows_grid(m->mhead.ntiles);
        a.part_v = m->part_v; a.part_i = m->part_i; a.nblk = grid; a.rlogits = m->r_logits;
        launch(m->cfg.profile, "head", k_head_rows<RT, EPI_PHEAD>, dim3(grid), dim3(256), 0, m->st, a);
        RaceArgs r{};
        r.part_v = m->part_v; r.part_i = m->part_i; r.nblk = grid; r.seq = m->seq; r.seq_stride = m->ctx + 1;
        r.words = m->words; r.words_stride = m->ctx + 1; r.pos = posp; r.plen = ctl + CTL_PLEN;
        r.pos_next = ctl + (m->par ? CTL_POS : CTL_POS1); r.nwords = ctl + CTL_NWORDS;
        if (race) {
            launch(m->cfg.profile, "race", k_race_rows, dim3(B), dim3(256), 0, m->st, r);
            m->par ^= 1;                             // the next step reads the slot this race writes
        }
    }
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// rec (batch 1): the step runs the kernels that record (sm_record_at's position)
// fused: batch 1 (m->fold), the race of the step before runs in this step's layer-0 qkv; race: the step ends
// with k_race1 (a run's last step; the other machines always race at the step's end)
static int launch_step(sm_machine* m, int parts = STEP_ALL, bool rec = false, bool fused = false, bool race = true) {
    if (m->kind == 1 && m->B > 1) {
        const int RT = (m->B + 15) / 16;
        if (RT == 1) return launch_step_pythia_batched<1>(m, parts, 0, nullptr, fused, race);
        if (RT == 2) return launch_step_pythia_batched<2>(m, parts, 0, nullptr, fused, race);
        if (RT == 3) return launch_step_pythia_batched<3>(m, parts, 0, nullptr, fused, race);
        return launch_step_pythia_batched<4>(m, parts, 0, nullptr, fused, race);
    }
    if (m->kind == 1) return launch_step_pythia(m, parts, rec);
    if (m->B > 1) {
        const int RT = (m->B + 15) / 16;
        if (RT == 1) return launch_step_batched<1>(m, parts, 0, nullptr, fused, race);
        if (RT == 2) return launch_step_batched<2>(m, parts, 0, nullptr, fused, race);
        if (RT == 3) return launch_step_batched<3>(m, parts, 0, nullptr, fused, race);
        return launch_step_batched<4>(m, parts, 0, nullptr, fused, race);
    }
    const Tables tb = m->T.tb();
    int* ctl = m->ctl;
    // the step's position slot.  With the race of the step before folded in, layer 0's qkv reads that step's slot
    // and writes the other one, which every later kernel of this step reads (the slots alternate step by step)
    const bool fold = m->fold && fused && parts == STEP_ALL;
    if (!m->fold || parts != STEP_ALL) race = true;
    int* const posA = ctl + (m->par ? CTL_POS1 : CTL_POS);
    int* const posp = fold ? ctl + (m->par ? CTL_POS : CTL_POS1) : posA;
    Race1Args rfold = race1_args(m);
    rfold.pos = posA; rfold.pos_next = posp;
    if (fold) m->par ^= 1;
    for (int l = 0; l < 12 && (parts & STEP_LAYERS); l++) {
        GemvArgs base{};
        base.tb = tb;
        base.pos = posp;
        base.rec_pos = ctl + CTL_RECPOS;
        const i64* Rin = l == 0 ? m->R0 : m->R;        // layer 0 reads the entering row (k_race1 / k_embed1 / PRO_RACE)
        // qkv: the stream's gauge, the product, power + bias (base2.py:105 gauged_bank(R, "qkv.l"))
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][0];
            a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
            a.X = Rin; a.Y = m->QKV;
            a.rx16 = m->r_x16 + (l * 4 + 0) * 3072; a.rexls = m->r_exls + (l * 4 + 0) * 2;
            a.rpile = m->r_pile + (l * 4 + 0) * 3072; a.rout = m->r_qkv + l * 2304;
            set_pf(a, m->bank[l][1], 2, grid2(m->bank[l][1]));
            if (l == 0 && fold) {       // the race of the step before, then the gauge of the row it feeds back
                a.pos = posA; a.race = rfold;
                gemv<768, 2, 4, PRO_RACE, EPI_GAUGED>(m, rec, "qkv.race", (P.ntiles + 3) / 4, a);
            } else {
                gemv<768, 2, 4, PRO_GAUGE, EPI_GAUGED>(m, rec, "qkv", (P.ntiles + 3) / 4, a);
            }
        }
        // attention (base2.py:85-100) on the KV cache of layer l
        {
            AttArgs a{};
            const size_t per = (size_t)m->B * m->ctx;
            a.QKV = m->QKV; a.K16 = m->K16 + l * per * 768; a.KM = m->KM + l * per * 12; a.EK = m->EK + l * per * 12; a.V = m->V + l * per * 768;
            a.V64 = m->V64 ? m->V64 + l * per * 768 : nullptr; a.VW = m->VW ? m->VW + l * per * 12 : nullptr;
            a.vbig = m->vbig ? m->vbig + (size_t)l * m->B * 12 : nullptr;
            a.out = m->att; a.pos = posp; a.ctx = m->ctx; a.tb = tb; a.err = ctl + CTL_ERR;
            a.rec_pos = ctl + CTL_RECPOS; a.ratt = m->r_att + l * 768;
            // proj: to16 of the attention row, product, plain shift + bias, added to R (base2.py:105; layer 0: to
            // the entering row)
            GemvArgs g = base;
            const DevPlate& P = m->bank[l][1];
            g.W = reinterpret_cast<const int4*>(P.W); g.we = P.e; g.bias = P.b; g.sw = P.sw; g.nout = P.nout; g.ntiles = P.ntiles;
            g.X = m->att; g.Y = m->R; g.Yb = Rin;
            g.rx16 = m->r_x16 + (l * 4 + 1) * 3072; g.rexls = m->r_exls + (l * 4 + 1) * 2;
            g.rpile = m->r_pile + (l * 4 + 1) * 3072; g.rout = m->r_resid + (l * 2 + 0) * 768;
            set_pf(g, m->bank[l][2], 4, grid4(m->bank[l][2]));
            attend1<0>(m, rec, a, l);
            if (m->att_long) {          // the attention's output row formed in proj's blocks
                g.aacc = m->aacc; g.ratt = m->r_att + l * 768;
                gemv<768, 2, 2, PRO_ATT, EPI_PLAIN_ADD>(m, rec, "proj", (P.ntiles + 1) / 2, g);
            } else {
                gemv<768, 2, 2, PRO_TO16, EPI_PLAIN_ADD>(m, rec, "proj", (P.ntiles + 1) / 2, g);
            }
        }
        // fc: gauge, product, gauged, edge (base2.py:106)
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][2];
            a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
            a.X = m->R; a.Y = m->hid;
            a.rx16 = m->r_x16 + (l * 4 + 2) * 3072; a.rexls = m->r_exls + (l * 4 + 2) * 2;
            a.rpile = m->r_pile + (l * 4 + 2) * 3072; a.rout = m->r_hid + l * 3072;
            set_pf(a, m->bank[l][3], 4, grid4(m->bank[l][3]));
            gemv<768, 2, 4, PRO_GAUGE, EPI_GAUGED_EDGE>(m, rec, "fc", (P.ntiles + 3) / 4, a);
        }
        // mproj: to16 of the hidden row (3072), product, plain, added to R (base2.py:106)
        {
            GemvArgs a = base;
            const DevPlate& P = m->bank[l][3];
            a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
            a.X = m->hid; a.Y = m->R; a.Yb = m->R;
            a.rx16 = m->r_x16 + (l * 4 + 3) * 3072; a.rexls = m->r_exls + (l * 4 + 3) * 2;
            a.rpile = m->r_pile + (l * 4 + 3) * 3072; a.rout = m->r_resid + (l * 2 + 1) * 768;
            if (l < 11) set_pf(a, m->bank[l + 1][0], 4, grid4(m->bank[l + 1][0]));
            else set_pf_head(m, a);
            gemv<3072, 1, 4, PRO_TO16, EPI_PLAIN_ADD>(m, rec, "mproj", (P.ntiles + 3) / 4, a);
        }
    }
    // head: gauge, product with the tied word table, power + standing amount, race (base2.py:107-114)
    if (parts & STEP_HEAD) {
        GemvArgs a{};
        a.tb = tb;
        a.pos = posp; a.rec_pos = ctl + CTL_RECPOS;
        const DevPlate& P = m->head;
        a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
        a.X = m->R;
        a.rx16 = m->r_hx16; a.rexls = m->r_hexls; a.rpile = m->r_hpile; a.rlogits = m->r_logits;
        a.part_v = m->part_v; a.part_i = m->part_i;      // each block's best; the race runs in k_race1
        if (m->cfg.top_read && !rec) {
            // the collapsing top read: the high-byte plane with each word's bounds, then the survivors' low
            // bytes and the race (a recorded step reads the full table, so that every logit is recorded)
            a.W = reinterpret_cast<const int4*>(m->top_hi);
            a.cand_j = m->cand_j; a.cand_h = m->cand_h; a.cand_c = m->cand_c; a.tx = m->top_x; a.tf = m->top_f;
            launch(m->cfg.profile, "head.top", k_gemv<768, HEAD_TC, HEAD_WPB, PRO_GAUGE, EPI_TOP1, 0, 0>, dim3(m->head_grid),
                   dim3(64 * HEAD_WPB), 0, m->st, a);
            TopArgs t{};
            t.r = race1_args(m);
            t.cap = HEAD_WPB * TOP_ITERS * HEAD_TC;
            t.cand_j = m->cand_j; t.cand_h = m->cand_h; t.cand_c = m->cand_c; t.tx = m->top_x; t.tf = m->top_f;
            t.lo = m->top_lo; t.we = P.e; t.bias = P.b; t.tb = tb;
            t.tn = m->top_n; t.tw = m->top_w; t.tpile = m->top_pile; t.tscore = m->top_score; t.tmax = TOP_RECORD;
            launch(m->cfg.profile, "race.top", k_race_top, dim3(1), dim3(256), 0, m->st, t);
        } else {
            gemv<768, HEAD_TC, HEAD_WPB, PRO_GAUGE, EPI_HEAD>(m, rec, "head", m->head_grid, a);
            if (race) launch_race1(m);
        }
    }
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// positions [0, npos) of every stream as passes of up to prefill_rows prompt rows, stream by stream (rows of one
// stream in position order, so a pass's keys and values at earlier positions are cached before it runs); then the
// device position moves to npos.  Nothing is recorded: the caller stops short of a recorded position.
static int run_prefill(sm_machine* m, int npos) {
    const int total = m->B * npos, chunk = m->cfg.prefill_rows;
    m->h_pfmap.resize(total);
    for (int s = 0; s < m->B; s++)
        for (int q = 0; q < npos; q++) m->h_pfmap[(size_t)s * npos + q] = s << 16 | q;
    HIP_TRY(hipMemcpyAsync(m->pfmap, m->h_pfmap.data(), (size_t)total * 4, hipMemcpyHostToDevice, m->st));
    for (int r0 = 0; r0 < total; r0 += chunk) {
        const int n = std::min(chunk, total - r0), RT = (n + 15) / 16;
        const int* map = m->pfmap + r0;
        int rc;
        if (m->kind == 1) {
            rc = RT == 1 ? launch_step_pythia_batched<1>(m, STEP_LAYERS, n, map)
               : RT == 2 ? launch_step_pythia_batched<2>(m, STEP_LAYERS, n, map)
               : RT == 3 ? launch_step_pythia_batched<3>(m, STEP_LAYERS, n, map)
                         : launch_step_pythia_batched<4>(m, STEP_LAYERS, n, map);
        } else {
            rc = RT == 1 ? launch_step_batched<1>(m, STEP_LAYERS, n, map)
               : RT == 2 ? launch_step_batched<2>(m, STEP_LAYERS, n, map)
               : RT == 3 ? launch_step_batched<3>(m, STEP_LAYERS, n, map)
                         : launch_step_batched<4>(m, STEP_LAYERS, n, map);
        }
        if (rc) return rc;
    }
    m->h_pfpos = npos;
    HIP_TRY(hipMemcpyAsync(m->ctl + (m->par ? CTL_POS1 : CTL_POS), &m->h_pfpos, 4, hipMemcpyHostToDevice, m->st));
    return SM_OK;
}

extern "C" int sm_create(const char* layout_dir, const sm_config* cfg, sm_machine** out) {
    if (!layout_dir || !out) return fail(SM_E_ARG, "sm_create: null argument");
    *out = nullptr;
    sm_config c{1, 1024, 1, 0, 16, 0, 0, 64, 0, 0, 2, 0, 0};
    if (cfg) c = *cfg;
    if (c.max_streams < 1 || c.max_streams > 64) return fail(SM_E_ARG, "sm_create: max_streams must be in [1, 64]");
    if (c.prefill_rows < 0 || c.prefill_rows > 64) return fail(SM_E_ARG, "sm_create: prefill_rows must be in [0, 64]");
    if (c.max_ctx <= 0) return fail(SM_E_ARG, "sm_create: max_ctx must be positive");
    // graphs of at most 16 steps, the largest that has run: a profiled run of a 127-step graph ended in a SIGSEGV
    // inside the profiled process, unexplained, so longer captures are refused rather than reached
    if (c.graph_steps < 0 || c.graph_steps > 16) return fail(SM_E_ARG, "sm_create: graph_steps must be in [0, 16]");
    if (c.att_split < -1) return fail(SM_E_ARG, "sm_create: att_split must be -1, 0 or a position");
    if (c.v64 < 0 || c.v64 > 1) return fail(SM_E_ARG, "sm_create: v64 must be 0 or 1");
    if (c.v64 && (c.float_stages & SM_FLOAT_ARRIVAL)) return fail(SM_E_ARG, "sm_create: the float arrival keeps no 64-bit values");
    const std::string dir = std::string(layout_dir) + "/";
    std::vector<char> mj;
    if (!read_file(dir + "manifest.json", mj)) return fail(SM_E_IO, "cannot read " + dir + "manifest.json");
    std::vector<BankInfo> banks;
    long long log768, eps40, alen;
    const std::string mtext(mj.begin(), mj.end());
    int rc = parse_manifest(mtext, banks, log768, eps40, alen);
    if (rc) return rc;
    const bool py = mtext.find("\"pythia\"") != std::string::npos;     // "kind": "pythia"
    long long rot = 0, half = 0, hs = 64;
    std::vector<std::pair<std::string, long long>> norms;
    if (py) {
        if (!json_int(mtext, 0, "rot", rot) || !json_int(mtext, 0, "half_log2_hs", half) || !json_int(mtext, 0, "hs", hs))
            return fail(SM_E_IO, "manifest.json: Pythia constants missing");
        if (hs != 64 || rot <= 0 || rot > 64 || rot % 2) return fail(SM_E_IO, "manifest.json: built for 12 heads of 64 and an even turned width");
        if ((rc = parse_norms(mtext, norms))) return rc;
    }
    // split digits: every plate and the word table come with a subtracted half (X.wsc), the digit being X.wc - X.wsc
    // (the Pythia machine's plates=built, foundation0/pythia_base2.py:44-46: finished - start, 17 bits a digit)
    long long splitv = 0;
    const bool split = py && json_int(mtext, 0, "split", splitv) && splitv != 0;
    if (split && (c.max_streams != 1 || c.prefill_rows != 0))
        return fail(SM_E_ARG, "sm_create: a layout of split digits (plates=built) runs with max_streams 1 and prefill_rows 0");
    if (c.inv && (py || c.max_streams != 1 || c.prefill_rows != 0))
        return fail(SM_E_ARG, "sm_create: the complement machine (inv) runs GPT-2 with max_streams 1 and prefill_rows 0");
    if (c.float_stages & ~(SM_FLOAT_GAUGE | SM_FLOAT_EDGE | SM_FLOAT_ARRIVAL | SM_FLOAT_TURN))
        return fail(SM_E_ARG, "sm_create: unknown float_stages bits");
    if (c.float_stages && (c.max_streams != 1 || c.prefill_rows != 0 || c.inv))
        return fail(SM_E_ARG, "sm_create: the float stages run with max_streams 1 and prefill_rows 0, without inv");
    if ((c.float_stages & SM_FLOAT_TURN) && !py) return fail(SM_E_ARG, "sm_create: turn=float is the Pythia machine's");
    if (c.top_read < 0 || c.top_read > 2) return fail(SM_E_ARG, "sm_create: top_read must be 0, 1 or 2");
    if (c.top_read == 2 && (py || c.max_streams != 1 || c.inv || c.float_stages)) c.top_read = 0;   // where it applies
    if (c.top_read == 1 && (py || c.max_streams != 1 || c.inv || c.float_stages))
        return fail(SM_E_ARG, "sm_create: the collapsing top read runs GPT-2 with max_streams 1, without inv or float stages");
    auto find = [&](const std::string& n) -> const BankInfo* {
        for (auto& b : banks) if (b.name == n) return &b;
        return nullptr;
    };
    sm_machine* m = new sm_machine();
    m->cfg = c;
    m->B = c.max_streams;
    m->RC = std::max(m->B, c.prefill_rows);
    m->kind = py ? 1 : 0;
    m->mode = (c.inv ? MODE_INV : 0) | (c.float_stages & SM_FLOAT_GAUGE ? MODE_FGAUGE : 0) |
              (c.float_stages & SM_FLOAT_EDGE ? MODE_FEDGE : 0) | (split ? MODE_SPLIT : 0);
    m->fturn = c.float_stages & SM_FLOAT_TURN;
    m->farr = c.float_stages & SM_FLOAT_ARRIVAL;
    // the spread attention: batch 1 with the integer arrival and turn
    if (m->B == 1 && !m->farr && !m->fturn && c.att_split != -1) m->att_split = c.att_split > 0 ? c.att_split : SM_ATT_SPLIT_AT;
    m->fold = m->B > 1 || (!py && m->mode == 0 && !m->farr && !c.top_read);
    const bool mfma = m->B > 1 || c.prefill_rows > 0;     // the MFMA banks: batched streams or prompt passes

    auto bail = [&](int code) { machine_free(m); return code; };
    {
        hipError_t e = hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking);
        if (e != hipSuccess) return bail(fail(SM_E_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e)));
    }
    // banks
    for (int l = 0; l < 12; l++) {
        for (int k = 0; k < 4; k++) {
            const std::string name = std::string(BANK[k]) + "." + std::to_string(l);
            const BankInfo* bi = find(name);
            if (!bi || bi->nin != NIN[k] || bi->nout != NOUT[k]) return bail(fail(SM_E_IO, "manifest.json: bank " + name + " missing or of the wrong shape"));
            std::vector<int16_t> w, w2; std::vector<int32_t> e; std::vector<i64> b;
            if ((rc = read_array(dir + name + ".wc", w, (size_t)NIN[k] * NOUT[k])) || (rc = read_array(dir + name + ".e", e, NOUT[k])) ||
                (rc = read_array(dir + name + ".b", b, NOUT[k])) ||
                (split && (rc = read_array(dir + name + ".wsc", w2, (size_t)NIN[k] * NOUT[k]))))
                return bail(rc);
            if (m->B == 1 && (rc = upload_plate(m->bank[l][k], w.data(), e.data(), b.data(), NIN[k], NOUT[k], TCOLS[k], c.inv,
                                                split ? w2.data() : nullptr)))
                return bail(rc);
            if (mfma && (rc = upload_mfma_plate(m->mbank[l][k], w.data(), e.data(), b.data(), NIN[k], NOUT[k]))) return bail(rc);
        }
    }
    const BankInfo* hb = find("head");
    if (!hb || hb->nin != 768 || hb->nout <= 0 || hb->nout > (1 << 24)) return bail(fail(SM_E_IO, "manifest.json: head bank missing or of the wrong shape"));
    m->vocab = (int)hb->nout;
    {   // the top read: every wave of its first stage finishes at most TOP_ITERS tiles, and its race reads at most
        // 512 blocks (top_read 2 falls back to the full read where the head grid does not allow it)
        const long long nt = (m->vocab + HEAD_TC - 1) / HEAD_TC, hg = c.head_grid > 0 ? c.head_grid : 512;
        const bool fits = hg <= 512 && hg * HEAD_WPB * TOP_ITERS >= nt;
        if (c.top_read == 2 && !fits) c.top_read = 0;
        if (c.top_read == 1 && !fits)
            return bail(fail(SM_E_ARG, "sm_create: the top read needs head_grid in [" +
                                           std::to_string((nt + HEAD_WPB * TOP_ITERS - 1) / (HEAD_WPB * TOP_ITERS)) + ", 512]"));
        m->cfg.top_read = c.top_read;
    }
    {
        std::vector<int16_t> w, w2; std::vector<int32_t> e; std::vector<i64> b;
        if ((rc = read_array(dir + "head.wc", w, (size_t)768 * m->vocab)) || (rc = read_array(dir + "head.e", e, m->vocab)) ||
            (split && (rc = read_array(dir + "head.wsc", w2, (size_t)768 * m->vocab))))
            return bail(rc);
        if (py) b.assign(m->vocab, 0);         // Pythia's head has no bias (foundation0/pythia_base2.py:159)
        else if ((rc = read_array(dir + "head.b", b, m->vocab))) return bail(rc);
        if (m->B == 1 && (rc = upload_plate(m->head, w.data(), e.data(), b.data(), 768, m->vocab, HEAD_TC, c.inv,
                                            split ? w2.data() : nullptr)))
            return bail(rc);
        if (c.top_read) {
            const std::vector<int8_t> hi = tile_hi_plane(w.data(), 768, m->vocab, HEAD_TC);
            const std::vector<uint8_t> lo = lo_plane(w.data(), 768, m->vocab);
            if ((rc = dalloc(&m->top_hi, hi.size())) || (rc = dalloc(&m->top_lo, lo.size()))) return bail(rc);
            if (hipMemcpy(m->top_hi, hi.data(), hi.size(), hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(m->top_lo, lo.data(), lo.size(), hipMemcpyHostToDevice) != hipSuccess)
                return bail(fail(SM_E_HIP, "upload the top read's planes"));
        }
        if (m->B > 1 && (rc = upload_mfma_plate(m->mhead, w.data(), e.data(), b.data(), 768, m->vocab))) return bail(rc);
    }
    // word and position tables
    if (py) {
        std::vector<int16_t> ew, ew2; std::vector<int32_t> ee; std::vector<i64> cs, sn;
        if ((rc = read_array(dir + "embed.wc", ew, (size_t)m->vocab * 768)) || (rc = read_array(dir + "embed.e", ee, m->vocab)) ||
            (rc = read_array(dir + "cos.bin", cs, (size_t)-1)) || (rc = read_array(dir + "sin.bin", sn, (size_t)-1)) ||
            (split && (rc = read_array(dir + "embed.wsc", ew2, (size_t)m->vocab * 768))))
            return bail(rc);
        if (split) {
            if ((rc = dalloc(&m->ew2, ew2.size()))) return bail(rc);
            if (hipMemcpy(m->ew2, ew2.data(), ew2.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
                return bail(fail(SM_E_HIP, "upload embed.wsc"));
        }
        const size_t r2 = (size_t)rot / 2;
        if (cs.empty() || cs.size() % r2 || sn.size() != cs.size()) return bail(fail(SM_E_IO, "cos.bin / sin.bin: not [positions][rot / 2]"));
        m->npos = (int)(cs.size() / r2);
        std::vector<int> c32(cs.size()), s32(sn.size());
        for (size_t i = 0; i < cs.size(); i++) {
            if (cs[i] < -(1 << 30) || cs[i] > (1 << 30) || sn[i] < -(1 << 30) || sn[i] > (1 << 30))
                return bail(fail(SM_E_IO, "cos.bin / sin.bin: a value past 2^30"));
            c32[i] = (int)cs[i]; s32[i] = (int)sn[i];
        }
        for (int v : ee) if (v < -80 || v > 40) return bail(fail(SM_E_IO, "embed.e: a power of two out of range"));
        if ((rc = dalloc(&m->ew, ew.size())) || (rc = dalloc(&m->ee, ee.size())) || (rc = dalloc(&m->cosT, c32.size())) ||
            (rc = dalloc(&m->sinT, s32.size())))
            return bail(rc);
        if (hipMemcpy(m->ew, ew.data(), ew.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m->ee, ee.data(), ee.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m->cosT, c32.data(), c32.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m->sinT, s32.data(), s32.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(SM_E_HIP, "upload embed / turns"));
        m->rot = (int)rot;
        if (m->fturn) {        // turn=float: the float64 cos and sin the layout wrote with numpy
            std::vector<double> cf, sf;
            if ((rc = read_array(dir + "cosf.bin", cf, cs.size())) || (rc = read_array(dir + "sinf.bin", sf, cs.size())))
                return bail(rc);
            if ((rc = dalloc(&m->cosF, cf.size())) || (rc = dalloc(&m->sinF, sf.size()))) return bail(rc);
            if (hipMemcpy(m->cosF, cf.data(), cf.size() * 8, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(m->sinF, sf.data(), sf.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
                return bail(fail(SM_E_HIP, "upload cosf / sinf"));
        }
        m->half = half;
        // the norms: gain on 16 places, offset at 2^-16, one power of two each
        auto norm = [&](const std::string& name, int*& g, i64*& b, int& ge) -> int {
            long long gev = 0;
            bool found = false;
            for (auto& nv : norms) if (nv.first == name) { gev = nv.second; found = true; }
            if (!found) return fail(SM_E_IO, "manifest.json: norm " + name + " missing");
            std::vector<int32_t> gh; std::vector<i64> bh;
            int r;
            if ((r = read_array(dir + name + ".g", gh, 768)) || (r = read_array(dir + name + ".b", bh, 768))) return r;
            const int gmax = split ? 65535 : 32767;      // (split digits: a difference of two 16-place gains)
            for (int v : gh) if (v < -gmax || v > gmax) return fail(SM_E_IO, name + ".g: a gain past " + (split ? "17" : "16") + " places");
            if (gev < -64 || gev > 16) return fail(SM_E_IO, name + ": gain power out of range");
            if ((r = dalloc(&g, (size_t)768)) || (r = dalloc(&b, (size_t)768))) return r;
            HIP_TRY(hipMemcpy(g, gh.data(), 768 * 4, hipMemcpyHostToDevice));
            HIP_TRY(hipMemcpy(b, bh.data(), 768 * 8, hipMemcpyHostToDevice));
            ge = (int)gev;
            return SM_OK;
        };
        for (int l = 0; l < 12; l++)
            for (int j = 0; j < 2; j++)
                if ((rc = norm((j ? "ln2." : "ln1.") + std::to_string(l), m->ng[l][j], m->nb[l][j], m->nge[l][j]))) return bail(rc);
        if ((rc = norm("lnf", m->fg, m->fb, m->fge))) return bail(rc);
    } else {
        std::vector<i64> wte, wpe;
        if ((rc = read_array(dir + "wte.bin", wte, (size_t)m->vocab * 768)) || (rc = read_array(dir + "wpe.bin", wpe, (size_t)-1))) return bail(rc);
        if (wpe.size() % 768 || wpe.empty()) return bail(fail(SM_E_IO, "wpe.bin: not a whole number of 768-wide rows"));
        m->npos = (int)(wpe.size() / 768);
        if ((rc = dalloc(&m->wte, wte.size())) || (rc = dalloc(&m->wpe, wpe.size()))) return bail(rc);
        if (hipMemcpy(m->wte, wte.data(), wte.size() * 8, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m->wpe, wpe.data(), wpe.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(SM_E_HIP, "upload wte/wpe"));
    }
    // tables
    {
        std::vector<i64> phi, arr, lg, ep;
        if ((rc = read_array(dir + "phi.bin", phi, 65536)) || (rc = read_array(dir + "arrival.bin", arr, (size_t)alen)) ||
            (rc = read_array(dir + "log2.bin", lg, 65536)) || (rc = read_array(dir + "exp2.bin", ep, 65536)))
            return bail(rc);
        if ((rc = tables_init(m->T, phi.data(), arr.data(), (int)alen, lg.data(), ep.data(), log768, eps40))) return bail(rc);
        m->ehalf = ep[(-m->half) & 0xFFFF];
        if (c.table_mode == 1 && !m->T.verified)
            return bail(fail(SM_E_IO, "sm_create: a table entry differs from its formula (base2_convert.py:48-61)"));
    }
    m->ctx = c.max_ctx < m->npos ? c.max_ctx : m->npos;
    m->head_grid = c.head_grid > 0 ? c.head_grid : 512;     // two blocks per CU (measured best)
    if (m->head_grid > 1024) return bail(fail(SM_E_ARG, "sm_create: head_grid at most 1024"));
    if (c.top_read) {
        const size_t cap = (size_t)HEAD_WPB * TOP_ITERS * HEAD_TC, g = m->head_grid;
        if ((rc = dalloc(&m->cand_j, g * cap)) || (rc = dalloc(&m->cand_h, g * cap)) || (rc = dalloc(&m->cand_c, g * cap)) ||
            (rc = dalloc(&m->top_x, (size_t)768)) || (rc = dalloc(&m->top_f, (size_t)4)) || (rc = dalloc(&m->top_n, (size_t)1)) ||
            (rc = dalloc(&m->top_w, (size_t)TOP_RECORD)) || (rc = dalloc(&m->top_pile, (size_t)TOP_RECORD)) ||
            (rc = dalloc(&m->top_score, (size_t)TOP_RECORD)))
            return bail(rc);
    }
    const size_t nparts = m->B == 1 ? (size_t)m->head_grid : (size_t)m->B * head_rows_grid((m->vocab + 15) / 16);
    // state
    const size_t B = m->B, ctx = m->ctx, RC = m->RC;
    const size_t nsets = m->kind == 1 && mfma ? 2 : 1;      // light-plane sets (the Pythia MFMA phases keep two)
    if ((rc = dalloc(&m->R, RC * 768)) || (rc = dalloc(&m->R0, 768)) || (rc = dalloc(&m->QKV, RC * 2304)) || (rc = dalloc(&m->att, RC * 768)) || (rc = dalloc(&m->attor, RC * 12)) ||
        (rc = dalloc(&m->hidor, RC * 192)) || (rc = dalloc(&m->sfacts, 4 * RC * 4)) ||
        (rc = dalloc(&m->hid, RC * 3072)) || (mfma && ((rc = dalloc(&m->att32, RC * 768)) || (rc = dalloc(&m->hid32, RC * 3072)))) || (rc = dalloc(&m->K16, 12 * B * ctx * 768)) || (rc = dalloc(&m->KM, 12 * B * ctx * 12)) ||
        (rc = dalloc(&m->EK, 12 * B * ctx * 12)) ||
        (rc = dalloc(&m->pfmap, B * ctx)) ||
        (rc = dalloc(&m->V, 12 * B * ctx * 768)) || (m->farr && (rc = dalloc(&m->KF, 12 * ctx * 768))) || (rc = dalloc(&m->seq, B * (ctx + 1))) || (rc = dalloc(&m->words, B * (ctx + 1))) ||
        (rc = dalloc(&m->ctl, (size_t)CTL_N)) || (rc = dalloc(&m->part_v, nparts)) ||
        (rc = dalloc(&m->part_i, nparts)) || (rc = dalloc(&m->r_x16, (size_t)12 * 4 * 3072)) ||
        (rc = dalloc(&m->planes, (size_t)4 * 48 * 3 * 1024 * nsets)) || (rc = dalloc(&m->rowinfo, RC * 8 * nsets)) ||
        (rc = dalloc(&m->part_acc, mfma ? (size_t)4 * RC * 3072 : (size_t)1)) ||
        (rc = dalloc(&m->r_exls, (size_t)12 * 4 * 2)) || (rc = dalloc(&m->r_pile, (size_t)12 * 4 * 3072)) ||
        (rc = dalloc(&m->r_qkv, (size_t)12 * 2304)) || (rc = dalloc(&m->r_att, (size_t)12 * 768)) ||
        (rc = dalloc(&m->r_hid, (size_t)12 * 3072)) || (rc = dalloc(&m->r_resid, (size_t)12 * 2 * 768)) ||
        (rc = dalloc(&m->r_hx16, 768)) || (rc = dalloc(&m->r_hexls, 2)) || (rc = dalloc(&m->r_hpile, (size_t)m->vocab)) ||
        (rc = dalloc(&m->r_logits, (size_t)m->vocab)) || (rc = dalloc(&m->r_gauge, (size_t)12 * 2 * 768)) ||
        (rc = dalloc(&m->r_fcpre, (size_t)12 * 3072)) || (rc = dalloc(&m->r_hgauge, (size_t)768)))
        return bail(rc);
    // rows with a value past 32 bits whole beside their low 32 bits (the float arrival keeps the int32 cache and its
    // error)
    if (!m->farr && ((rc = dalloc(&m->V64, 12 * B * ctx * 768)) || (rc = dalloc(&m->VW, 12 * B * ctx * 12)) ||
                     (rc = dalloc(&m->vbig, 12 * B * 12))))
        return bail(rc);
    if (m->att_split >= 0) {
        m->ncm = (int)((ctx + ACH_SPLIT - 1) / ACH_SPLIT);
        if ((rc = dalloc(&m->asc, 12 * ctx)) || (rc = dalloc(&m->acm, (size_t)12 * m->ncm)) ||
            (rc = dalloc(&m->aacc, (size_t)12 * ACC_W)))
            return bail(rc);
    }
    if (hipMemset(m->planes, 0, (size_t)4 * 48 * 3 * 1024 * nsets) != hipSuccess || hipMemset(m->rowinfo, 0, RC * 32 * nsets) != hipSuccess)
        return bail(fail(SM_E_HIP, "hipMemset planes"));
    if (hipHostMalloc(&m->hpin, (CTL_N + B * (ctx + 1)) * sizeof(int), hipHostMallocDefault) != hipSuccess) {
        m->hpin = nullptr;
        return bail(fail(SM_E_OOM, "hipHostMalloc: the generate readback buffer"));
    }
    m->prompts.assign(B, {});
    m->gsteps = c.graph_steps > 0 ? c.graph_steps : 16;
    if ((rc = sm_reset(m))) return bail(rc);
    *out = m;
    return SM_OK;
}

extern "C" int sm_destroy(sm_machine* m) {
    if (m) {
        (void)hipStreamSynchronize(m->st);
        machine_free(m);
    }
    return SM_OK;
}

extern "C" int sm_reset(sm_machine* m) {
    if (!m) return fail(SM_E_ARG, "sm_reset: null machine");
    const size_t B = m->B, ctx = m->ctx;
    HIP_TRY(hipMemsetAsync(m->ctl, 0, CTL_N * 4, m->st));
    int rp = -1;
    HIP_TRY(hipMemcpyAsync(m->ctl + CTL_RECPOS, &rp, 4, hipMemcpyHostToDevice, m->st));
    HIP_TRY(hipMemsetAsync(m->K16, 0, 12 * B * ctx * 768 * 2, m->st));
    HIP_TRY(hipMemsetAsync(m->KM, 0, 12 * B * ctx * 12 * 8, m->st));
    HIP_TRY(hipMemsetAsync(m->EK, 0, 12 * B * ctx * 12 * 4, m->st));
    HIP_TRY(hipMemsetAsync(m->V, 0, 12 * B * ctx * 768 * 4, m->st));
    // every head reads its values at 32 bits until one past 32 bits is stored (v64 = 1: whole from the start)
    if (m->vbig) HIP_TRY(hipMemsetAsync(m->vbig, m->cfg.v64 ? 1 : 0, 12 * B * 12 * 4, m->st));
    if (m->VW) HIP_TRY(hipMemsetAsync(m->VW, 0, 12 * B * ctx * 12 * 4, m->st));
    HIP_TRY(hipMemsetAsync(m->seq, 0, B * (ctx + 1) * 4, m->st));
    HIP_TRY(hipMemsetAsync(m->words, 0, B * (ctx + 1) * 4, m->st));
    HIP_TRY(hipMemsetAsync(m->R, 0, (size_t)m->RC * 768 * 8, m->st));
    HIP_TRY(hipMemsetAsync(m->R0, 0, 768 * 8, m->st));
    HIP_TRY(hipStreamSynchronize(m->st));
    m->h_plen = m->h_pos = m->h_words = 0;
    m->h_recpos = -1;
    m->par = 0;
    for (auto& p : m->prompts) p.clear();
    return SM_OK;
}

extern "C" int sm_prefill(sm_machine* m, int32_t stream, const int32_t* ids, int32_t n) {
    if (!m || !ids) return fail(SM_E_ARG, "sm_prefill: null argument");
    if (stream < 0 || stream >= m->B) return fail(SM_E_ARG, "sm_prefill: stream out of range");
    if (m->h_pos != 0) return fail(SM_E_STATE, "sm_prefill: the machine has already run; call sm_reset first");
    if (n <= 0 || n > m->ctx) return fail(SM_E_CTX, "sm_prefill: prompt length must be in [1, max_ctx]");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->vocab) return fail(SM_E_ARG, "sm_prefill: token id out of range");
    m->prompts[stream].assign(ids, ids + n);
    HIP_TRY(hipMemcpy(m->seq + (size_t)stream * (m->ctx + 1), ids, (size_t)n * 4, hipMemcpyHostToDevice));
    return SM_OK;
}

extern "C" int sm_record_at(sm_machine* m, int32_t pos) {
    if (!m) return fail(SM_E_ARG, "sm_record_at: null machine");
    HIP_TRY(hipMemcpy(m->ctl + CTL_RECPOS, &pos, 4, hipMemcpyHostToDevice));
    m->h_recpos = pos;
    return SM_OK;
}

// capture n consecutive launch sequences (parts of a step) into graph slot `which`
// (for the position slot the next step reads; capturing launches nothing, so the slot is put back)
static int capture(sm_machine* m, int which, int n, int parts) {
    const int p0 = m->par;
    if (m->gexec[which][p0]) return SM_OK;
    HIP_TRY(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
    int rc = SM_OK;
    // (a run: its first step takes the entering row already written, the later ones fold in the race of the step
    // before, and the last one races)
    for (int s = 0; s < n && !rc; s++) rc = launch_step(m, parts, false, s > 0, s == n - 1);
    m->gflip[which] = m->par != p0;
    m->par = p0;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m->st, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return fail(SM_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    m->graph[which][p0] = g;
    HIP_TRY(hipGraphInstantiate(&m->gexec[which][p0], g, nullptr, nullptr, 0));
    return SM_OK;
}
// replay graph slot `which` from the current position slot
static int replay(sm_machine* m, int which, int n, int parts) {
    int rc;
    if ((rc = capture(m, which, n, parts))) return rc;
    HIP_TRY(hipGraphLaunch(m->gexec[which][m->par], m->st));
    m->par ^= (int)m->gflip[which];
    return SM_OK;
}

// n whole decode steps of one attention structure: replayed from captured graphs, or launched one by one (always so
// with profile = 1, whose launches each carry their event pair)
static int queue_run(sm_machine* m, int steps) {
    int rc;
    const int g = m->att_long ? 4 : 0;
    if (m->cfg.use_graph && !m->cfg.profile) {
        for (; steps >= m->gsteps; steps -= m->gsteps)
            if ((rc = replay(m, g, m->gsteps, STEP_ALL))) return rc;
        for (; steps > 0; steps--)
            if ((rc = replay(m, g + 1, 1, STEP_ALL))) return rc;
    } else {
        for (int s = 0; s < steps; s++)
            if ((rc = launch_step(m, STEP_ALL, false, s > 0, s == steps - 1))) return rc;
    }
    return SM_OK;
}
// n decode steps from position pos: those before the split position with the one-block attention, the rest with
// the attention spread over chunks of positions
static int queue_steps(sm_machine* m, int steps, int pos) {
    int rc;
    if (m->att_split >= 0 && pos < m->att_split && steps > 0) {
        const int n = std::min(steps, m->att_split - pos);
        m->att_long = false;
        if ((rc = queue_run(m, n))) return rc;
        steps -= n;
        pos += n;
    }
    m->att_long = m->att_split >= 0 && pos >= m->att_split;
    return steps > 0 ? queue_run(m, steps) : SM_OK;
}

// n decode steps from position pos0.  At batch 1 the step at the recorded position runs on its own with the
// kernels that record (the others read no record position); the batched kernels check it themselves.
static int run_steps(sm_machine* m, int n, int pos0) {
    const int rp = m->B == 1 ? m->h_recpos : -1;
    int rc;
    if (rp >= pos0 && rp < pos0 + n) {
        if ((rc = queue_steps(m, rp - pos0, pos0))) return rc;
        m->att_long = m->att_split >= 0 && rp >= m->att_split;
        if ((rc = launch_step(m, STEP_ALL, true))) return rc;
        return queue_steps(m, pos0 + n - rp - 1, rp + 1);
    }
    return queue_steps(m, n, pos0);
}

extern "C" int sm_generate(sm_machine* m, int32_t n_words, int32_t* out) {
    if (!m) return fail(SM_E_ARG, "sm_generate: null machine");
    if (n_words <= 0) return fail(SM_E_ARG, "sm_generate: n_words must be positive");
    const bool first = m->h_pos == 0;
    if (first) {
        size_t n = m->prompts[0].size();
        for (int b = 0; b < m->B; b++)
            if (m->prompts[b].empty() || m->prompts[b].size() != n) return fail(SM_E_STATE, "sm_generate: every stream needs a prompt of the same length");
        m->h_plen = (int)n;
    }
    const int target = m->h_words + n_words;
    if (m->h_plen - 1 + target > m->ctx) return fail(SM_E_CTX, "sm_generate: prompt + words would pass max_ctx");
    int rc;
    if (first) {
        HIP_TRY(hipMemcpyAsync(m->ctl + CTL_PLEN, &m->h_plen, 4, hipMemcpyHostToDevice, m->st));
        // the prompt's positions but its last in passes of rows (not past a recorded position)
        int npos = m->h_plen - 1;
        if (m->h_recpos >= 0 && m->h_recpos < npos) npos = m->h_recpos;
        if (m->cfg.prefill_rows > 0 && npos > 0) {
            if ((rc = run_prefill(m, npos))) return rc;
            m->h_pos = npos;
        }
    }
    // batch 1: the first step's entering row (later steps' rows are written by the race of the step before)
    if (first && m->B == 1) launch_embed1(m);
    const int total = (m->h_plen - 1 + target) - m->h_pos;
    if ((rc = run_steps(m, total, m->h_pos))) return rc;
    // the control block and every stream's new words into pinned host memory, queued behind the steps, then one
    // wait (in place of a synchronous copy per stream)
    HIP_TRY(hipMemcpyAsync(m->hpin, m->ctl, CTL_N * sizeof(int), hipMemcpyDeviceToHost, m->st));
    HIP_TRY(hipMemcpy2DAsync(m->hpin + CTL_N, (size_t)n_words * 4, m->words + (target - n_words), (size_t)(m->ctx + 1) * 4,
                             (size_t)n_words * 4, (size_t)m->B, hipMemcpyDeviceToHost, m->st));
    HIP_TRY(hipStreamSynchronize(m->st));
    const int* ctl = m->hpin;
    m->h_pos += total;
    m->h_words = target;
    if (ctl[m->par ? CTL_POS1 : CTL_POS] != m->h_pos) return fail(SM_E_STATE, "sm_generate: device position disagrees with the host");
    if (ctl[CTL_ERR] & SM_ERR_V32)
        return fail(SM_E_OVERFLOW, "sm_generate: an attention value left 32 bits (the float arrival's value cache holds int32)");
    if (ctl[CTL_ERR] & SM_ERR_RANGE)
        return fail(SM_E_OVERFLOW, "sm_generate: a value passed a bound the reference asserts (turn input 2^31, attention sum 2^62)");
    std::memcpy(out, m->hpin + CTL_N, (size_t)m->B * n_words * sizeof(int));
    // a profiled machine folds its event pairs into the per-kernel sums now, so that their events are reused by the
    // next call instead of piling up over a long run
    if (m->cfg.profile && (rc = kt_fold())) return rc;
    return SM_OK;
}

extern "C" int sm_profile(sm_machine* m, int64_t* n_heads, double* head_us, int32_t clear) {
    if (!m) return fail(SM_E_ARG, "sm_profile: null machine");
    int rc;
    if ((rc = kt_fold())) return rc;
    std::lock_guard<std::mutex> lock(g_kt.mu);
    long long n = 0;
    double us = 0.0;
    for (size_t i = 0; i < g_kt.names.size(); i++)
        if (g_kt.names[i] == "head" || g_kt.names[i] == "head.top") { n += g_kt.n[i]; us += g_kt.us[i]; }
    if (n_heads) *n_heads = n;
    if (head_us) *head_us = us;
    if (clear)
        for (size_t i = 0; i < g_kt.names.size(); i++) { g_kt.n[i] = 0; g_kt.us[i] = 0.0; g_kt.syms[i].clear(); }
    return SM_OK;
}

extern "C" int sm_profile_stages(int32_t on) {
    g_kt.stages = on != 0;
    return SM_OK;
}

extern "C" int sm_profile_kernels(char* names, int32_t names_bytes, int64_t* launches, double* total_us, int32_t max,
                                  int32_t* n, int32_t clear) {
    if (!names || names_bytes <= 0 || !launches || !total_us || max < 0 || !n) return fail(SM_E_ARG, "sm_profile_kernels: arguments");
    int rc;
    if ((rc = kt_fold())) return rc;
    std::lock_guard<std::mutex> lock(g_kt.mu);
    std::string all;
    int k = 0;
    for (size_t i = 0; i < g_kt.names.size() && k < max; i++) {
        if (!g_kt.n[i]) continue;
        all += g_kt.names[i];
        const std::string* top = nullptr;                 // the symbol with the most launches under this name
        long long most = -1;
        for (const auto& kv : g_kt.syms[i])
            if (kv.second > most) { most = kv.second; top = &kv.first; }
        all += '\t';
        all += top ? *top : std::string("?");
        all += '\n';
        launches[k] = g_kt.n[i];
        total_us[k] = g_kt.us[i];
        k++;
    }
    if ((int64_t)all.size() + 1 > names_bytes) return fail(SM_E_ARG, "sm_profile_kernels: names buffer too small");
    std::memcpy(names, all.c_str(), all.size() + 1);
    *n = k;
    if (clear)
        for (size_t i = 0; i < g_kt.names.size(); i++) { g_kt.n[i] = 0; g_kt.us[i] = 0.0; g_kt.syms[i].clear(); }
    return SM_OK;
}

extern "C" int sm_read(sm_machine* m, int32_t what, int32_t layer, int32_t stream, int32_t pos, void* dst, size_t bytes) {
    if (!m || !dst) return fail(SM_E_ARG, "sm_read: null argument");
    if (stream < 0 || stream >= m->B) return fail(SM_E_ARG, "sm_read: stream out of range");
    const size_t B = m->B, ctx = m->ctx;
    const void* src = nullptr;
    size_t need = 0;
    auto kv_ok = [&]() { return layer >= 0 && layer < 12 && pos >= 0 && pos < m->ctx; };
    switch (what) {
        case SM_READ_V64: {
            // one position's values whole: a head's row from the 64-bit copy where the row is there, else its
            // 32-bit row widened
            if (!kv_ok()) return fail(SM_E_ARG, "sm_read: layer/pos");
            if (!m->V64) return fail(SM_E_STATE, "sm_read: this machine keeps no 64-bit values (float arrival)");
            if (bytes != 12 * 512) return fail(SM_E_ARG, "sm_read: expected 6144 bytes");
            const size_t h0 = ((size_t)layer * B + stream) * 12 * ctx + pos;
            int vw[12], v32[12 * 64];
            HIP_TRY(hipStreamSynchronize(m->st));
            HIP_TRY(hipMemcpy2D(dst, 512, m->V64 + h0 * 64, ctx * 512, 512, 12, hipMemcpyDeviceToHost));
            HIP_TRY(hipMemcpy2D(v32, 256, m->V + h0 * 64, ctx * 256, 256, 12, hipMemcpyDeviceToHost));
            HIP_TRY(hipMemcpy2D(vw, 4, m->VW + h0, ctx * 4, 4, 12, hipMemcpyDeviceToHost));
            int64_t* o = static_cast<int64_t*>(dst);
            for (int h = 0; h < 12; h++)
                if (!vw[h])
                    for (int d = 0; d < 64; d++) o[h * 64 + d] = v32[h * 64 + d];
            return SM_OK;
        }
        case SM_READ_K16: case SM_READ_EK: case SM_READ_V: {
            // one position's row, gathered from the 12 heads of the head-major cache
            if (!kv_ok()) return fail(SM_E_ARG, "sm_read: layer/pos");
            const size_t h0 = ((size_t)layer * B + stream) * 12 * ctx + pos;     // head 0's slot
            const bool ek = what == SM_READ_EK;
            const size_t w = ek ? 4 : 256;
            if (bytes != 12 * w) return fail(SM_E_ARG, "sm_read: expected " + std::to_string(12 * w) + " bytes");
            HIP_TRY(hipStreamSynchronize(m->st));
            if (what == SM_READ_K16) {      // int16 rows and their +32768 masks back to the keys' int32 values
                int16_t k[12][64];
                uint64_t km[12];
                HIP_TRY(hipMemcpy2D(k, 128, m->K16 + h0 * 64, ctx * 128, 128, 12, hipMemcpyDeviceToHost));
                HIP_TRY(hipMemcpy2D(km, 8, m->KM + h0, ctx * 8, 8, 12, hipMemcpyDeviceToHost));
                int32_t* out = static_cast<int32_t*>(dst);
                for (int h = 0; h < 12; h++)
                    for (int d = 0; d < 64; d++) out[h * 64 + d] = (int32_t)k[h][d] + (int32_t)((km[h] >> d) & 1);
                return SM_OK;
            }
            const void* s0 = ek ? (const void*)(m->EK + h0) : (const void*)(m->V + h0 * 64);
            HIP_TRY(hipMemcpy2D(dst, w, s0, ctx * w, w, 12, hipMemcpyDeviceToHost));
            return SM_OK;
        }
        case SM_READ_RESID: src = m->R + (size_t)stream * 768; need = 768 * 8; break;
        case SM_READ_SEQ: src = m->seq + (size_t)stream * (ctx + 1); need = (ctx + 1) * 4; break;
        case SM_READ_REC_X16: src = m->r_x16; need = 12 * 4 * 3072 * 8; break;
        case SM_READ_REC_EXLS: src = m->r_exls; need = 12 * 4 * 2 * 8; break;
        case SM_READ_REC_PILE: src = m->r_pile; need = 12 * 4 * 3072 * 8; break;
        case SM_READ_REC_QKV: src = m->r_qkv; need = 12 * 2304 * 8; break;
        case SM_READ_REC_ATT: src = m->r_att; need = 12 * 768 * 8; break;
        case SM_READ_REC_HID: src = m->r_hid; need = 12 * 3072 * 8; break;
        case SM_READ_REC_RESID: src = m->r_resid; need = 12 * 2 * 768 * 8; break;
        case SM_READ_REC_HX16: src = m->r_hx16; need = 768 * 8; break;
        case SM_READ_REC_HEXLS: src = m->r_hexls; need = 2 * 8; break;
        case SM_READ_REC_HPILE: src = m->r_hpile; need = (size_t)m->vocab * 8; break;
        case SM_READ_REC_LOGITS: src = m->r_logits; need = (size_t)m->vocab * 8; break;
        case SM_READ_REC_GAUGE: src = m->r_gauge; need = 12 * 2 * 768 * 8; break;
        case SM_READ_REC_FCPRE: src = m->r_fcpre; need = 12 * 3072 * 8; break;
        case SM_READ_REC_HGAUGE: src = m->r_hgauge; need = 768 * 8; break;
        case SM_READ_TOP: {
            if (!m->top_n) return fail(SM_E_STATE, "sm_read: the machine has no top read");
            if (bytes != (1 + 3 * TOP_RECORD) * 8) return fail(SM_E_ARG, "sm_read: expected " + std::to_string((1 + 3 * TOP_RECORD) * 8) + " bytes");
            HIP_TRY(hipStreamSynchronize(m->st));
            int n = 0;
            std::vector<int> w(TOP_RECORD);
            std::vector<i64> pl(TOP_RECORD), sc(TOP_RECORD);
            HIP_TRY(hipMemcpy(&n, m->top_n, 4, hipMemcpyDeviceToHost));
            HIP_TRY(hipMemcpy(w.data(), m->top_w, TOP_RECORD * 4, hipMemcpyDeviceToHost));
            HIP_TRY(hipMemcpy(pl.data(), m->top_pile, TOP_RECORD * 8, hipMemcpyDeviceToHost));
            HIP_TRY(hipMemcpy(sc.data(), m->top_score, TOP_RECORD * 8, hipMemcpyDeviceToHost));
            i64* out = static_cast<i64*>(dst);
            out[0] = n;
            for (int k = 0; k < TOP_RECORD; k++) { out[1 + 3 * k] = w[k]; out[2 + 3 * k] = pl[k]; out[3 + 3 * k] = sc[k]; }
            return SM_OK;
        }
        default: return fail(SM_E_ARG, "sm_read: unknown array");
    }
    if (bytes != need) return fail(SM_E_ARG, "sm_read: expected " + std::to_string(need) + " bytes");
    HIP_TRY(hipStreamSynchronize(m->st));
    HIP_TRY(hipMemcpy(dst, src, need, hipMemcpyDeviceToHost));
    return SM_OK;
}

extern "C" int sm_model_kind(const sm_machine* m) {
    if (!m) return fail(SM_E_ARG, "sm_model_kind: null machine");
    return m->kind;
}

extern "C" int sm_top_read(const sm_machine* m) {
    if (!m) return fail(SM_E_ARG, "sm_top_read: null machine");
    return m->cfg.top_read ? 1 : 0;
}

extern "C" int sm_info(const sm_machine* m, int32_t* vocab, int32_t* max_ctx, int32_t* max_streams, int32_t* n_pos,
                       int32_t* tables_verified) {
    if (!m) return fail(SM_E_ARG, "sm_info: null machine");
    if (tables_verified) *tables_verified = m->T.verified;
    if (vocab) *vocab = m->vocab;
    if (max_ctx) *max_ctx = m->ctx;
    if (max_streams) *max_streams = m->B;
    if (n_pos) *n_pos = m->npos;
    return SM_OK;
}

// ---------------------------------------------------------------------------------------------------------
// stage entry points
extern "C" int sm_tables_create(const int64_t* phi, const int64_t* arrival, int32_t alen, const int64_t* log2t,
                                const int64_t* exp2t, int64_t log2_768, int64_t eps40, sm_tables** out) {
    if (!phi || !arrival || !log2t || !exp2t || !out) return fail(SM_E_ARG, "sm_tables_create: null argument");
    sm_tables* t = new sm_tables();
    int rc = tables_init(*t, (const i64*)phi, (const i64*)arrival, alen, (const i64*)log2t, (const i64*)exp2t, log2_768, eps40);
    if (rc) { tables_free(*t); delete t; return rc; }
    *out = t;
    return SM_OK;
}

extern "C" int sm_tables_verified(const sm_tables* t) {
    if (!t) return fail(SM_E_ARG, "sm_tables_verified: null tables");
    return t->verified ? 1 : 0;
}

extern "C" int sm_tables_destroy(sm_tables* t) {
    if (t) { tables_free(*t); delete t; }
    return SM_OK;
}

static inline int blocks_for(int64_t n, int per) { return (int)((n + per - 1) / per); }

extern "C" int sm_stage_rshift(const int64_t* x, const int64_t* s, int64_t* out, int64_t n, void* stream) {
    if (n < 0 || (n > 0 && (!x || !s || !out))) return fail(SM_E_ARG, "sm_stage_rshift: arguments");
    if (n) launch(g_kt.stages, "stage.rshift", k_stage_rshift, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, (const i64*)x, (const i64*)s, (i64*)out, n);
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_log2fix(const sm_tables* t, const int64_t* v, int64_t* out, int64_t n, void* stream) {
    if (!t || n < 0 || (n > 0 && (!v || !out))) return fail(SM_E_ARG, "sm_stage_log2fix: arguments");
    if (n) launch(g_kt.stages, "stage.log2fix", k_stage_log2fix, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, (const i64*)v, (i64*)out, n, t->tb());
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_power(const sm_tables* t, const int64_t* x, const int64_t* F, int64_t* out, int64_t n, void* stream) {
    if (!t || n < 0 || (n > 0 && (!x || !F || !out))) return fail(SM_E_ARG, "sm_stage_power: arguments");
    if (n) launch(g_kt.stages, "stage.power", k_stage_power, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, (const i64*)x, (const i64*)F, (i64*)out, n, t->tb());
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_edge(const sm_tables* t, const int64_t* h, int64_t* out, int64_t n, void* stream) {
    if (!t || n < 0 || (n > 0 && (!h || !out))) return fail(SM_E_ARG, "sm_stage_edge: arguments");
    if (n) launch(g_kt.stages, "stage.edge", k_stage_edge, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, (const i64*)h, (i64*)out, n, t->tb());
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_to16(const int64_t* X, int32_t rows, int32_t n, int64_t* x16, int64_t* ex, void* stream) {
    if (rows < 0 || n <= 0 || (rows > 0 && (!X || !x16 || !ex))) return fail(SM_E_ARG, "sm_stage_to16: arguments");
    if (rows) launch(g_kt.stages, "stage.to16", k_stage_rows, dim3(rows), dim3(NTHR), 0, (hipStream_t)stream, (const i64*)X, n, 0, (i64*)x16, (i64*)ex, nullptr, Tables{});
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_gauge_log(const sm_tables* t, const int64_t* R, int32_t rows, int64_t* x16, int64_t* ex, int64_t* LS, void* stream) {
    if (!t || rows < 0 || (rows > 0 && (!R || !x16 || !ex || !LS))) return fail(SM_E_ARG, "sm_stage_gauge_log: arguments");
    if (rows) launch(g_kt.stages, "stage.gauge_log", k_stage_rows, dim3(rows), dim3(NTHR), 0, (hipStream_t)stream, (const i64*)R, 768, 1, (i64*)x16, (i64*)ex, (i64*)LS, t->tb());
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_race(const int64_t* v, int64_t n, int64_t* out_index, void* stream) {
    if (n <= 0 || !v || !out_index) return fail(SM_E_ARG, "sm_stage_race: arguments");
    launch(g_kt.stages, "stage.race", k_stage_race, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const i64*)v, n, (i64*)out_index);
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
extern "C" int sm_stage_attend(const sm_tables* t, const int64_t* qkv, int16_t* k16, int64_t* km, int32_t* ek, int32_t* v,
                               int32_t pos, int32_t ctx, int64_t* out, void* stream) {
    if (!t || !qkv || !k16 || !km || !ek || !v || !out || ctx <= 0 || pos < 0 || pos >= ctx || ctx > 8192)
        return fail(SM_E_ARG, "sm_stage_attend: arguments");
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemcpyAsync(t->scratch, &pos, 4, hipMemcpyHostToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));
    AttArgs a{};
    a.QKV = (const i64*)qkv; a.K16 = k16; a.KM = (i64*)km; a.EK = ek; a.V = v; a.out = (i64*)out; a.pos = t->scratch; a.ctx = ctx;
    a.tb = t->tb(); a.err = t->scratch + 1;
    launch(g_kt.stages, "stage.attend", k_attend<0, 1, 0>, dim3(12, 1), dim3(NTHR), (size_t)ctx * 12, s, a);
    HIP_TRY(hipGetLastError());
    int err = 0;
    HIP_TRY(hipMemcpyAsync(&err, t->scratch + 1, 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (err & SM_ERR_V32) {
        HIP_TRY(hipMemset(t->scratch + 1, 0, 4));
        return fail(SM_E_OVERFLOW, "sm_stage_attend: a value left 32 bits");
    }
    return SM_OK;
}

// the same attention spread over chunks of 64 positions, the batch-1 machine's kernels for positions from its split
// position on (sm_attend_split.hip)
#define SM_STAGE_ATT_CTX 8192
extern "C" int sm_stage_attend_split(const sm_tables* t, const int64_t* qkv, int16_t* k16, int64_t* km, int32_t* ek,
                                     int32_t* v, int32_t pos, int32_t ctx, int64_t* out, void* stream) {
    if (!t || !qkv || !k16 || !km || !ek || !v || !out || ctx <= 0 || pos < 0 || pos >= ctx || ctx > SM_STAGE_ATT_CTX)
        return fail(SM_E_ARG, "sm_stage_attend_split: arguments");
    sm_tables* tt = const_cast<sm_tables*>(t);
    const int ncm = (SM_STAGE_ATT_CTX + ACH_SPLIT - 1) / ACH_SPLIT;
    if (!tt->asc) {
        int rc;
        if ((rc = dalloc(&tt->asc, (size_t)12 * SM_STAGE_ATT_CTX)) || (rc = dalloc(&tt->acm, (size_t)12 * ncm)) ||
            (rc = dalloc(&tt->aacc, (size_t)12 * ACC_W))) {
            hfree(tt->asc); hfree(tt->acm); hfree(tt->aacc);
            tt->asc = tt->acm = tt->aacc = nullptr;
            return rc;
        }
    }
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemcpyAsync(t->scratch, &pos, 4, hipMemcpyHostToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));
    AttArgs a{};
    a.QKV = (const i64*)qkv; a.K16 = k16; a.KM = (i64*)km; a.EK = ek; a.V = v; a.out = (i64*)out; a.pos = t->scratch; a.ctx = ctx;
    a.tb = t->tb(); a.err = t->scratch + 1;
    a.asc = tt->asc; a.acm = tt->acm; a.aacc = tt->aacc; a.ncm = ncm;
    const dim3 grid(12, (ctx + ACH_SPLIT - 1) / ACH_SPLIT);
    const bool timed = g_kt.stages;
    launch(timed, "stage.attend.scores", k_att_scores<0>, grid, dim3(256), 0, s, a);
    launch(timed, "stage.attend.mix", k_att_mix<0, 0>, grid, dim3(256), 0, s, a);
    launch(timed, "stage.attend.finish", k_att_finish<0, 0>, dim3(12), dim3(64), 0, s, a);
    HIP_TRY(hipGetLastError());
    int err = 0;
    HIP_TRY(hipMemcpyAsync(&err, t->scratch + 1, 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (err & SM_ERR_V32) {
        HIP_TRY(hipMemset(t->scratch + 1, 0, 4));
        return fail(SM_E_OVERFLOW, "sm_stage_attend_split: a value left 32 bits");
    }
    return SM_OK;
}

extern "C" int sm_stage_attend_rows(const sm_tables* t, const int64_t* qkv, int32_t rows, int16_t* k16, int64_t* km,
                                    int32_t* ek, int32_t* v, int32_t pos, int32_t ctx, int64_t* out, void* stream) {
    if (!t || !qkv || !k16 || !km || !ek || !v || !out || rows <= 0 || rows > 1024 || ctx <= 0 || pos < 0 || pos >= ctx ||
        ctx > 8192)
        return fail(SM_E_ARG, "sm_stage_attend_rows: arguments");
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemcpyAsync(t->scratch, &pos, 4, hipMemcpyHostToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));
    AttArgs a{};
    a.QKV = (const i64*)qkv; a.K16 = k16; a.KM = (i64*)km; a.EK = ek; a.V = v; a.out = (i64*)out; a.pos = t->scratch; a.ctx = ctx;
    a.tb = t->tb(); a.err = t->scratch + 1;
    launch(g_kt.stages, "stage.attend_rows", k_attend<0, 0, 1>, dim3(12, rows), dim3(NTHR), (size_t)ctx * 12, s, a);      // the batched machine's kernel
    HIP_TRY(hipGetLastError());
    int err = 0;
    HIP_TRY(hipMemcpyAsync(&err, t->scratch + 1, 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (err & SM_ERR_V32) {
        HIP_TRY(hipMemset(t->scratch + 1, 0, 4));
        return fail(SM_E_OVERFLOW, "sm_stage_attend_rows: a value left 32 bits");
    }
    return SM_OK;
}

// tile_cols > 0: a GEMV plate (one light row per product); tile_cols == 0: an MFMA plate (rows of lights) with
// its own light planes and row sums
struct sm_plate {
    DevPlate P;
    MfmaPlate M;
    bool mfma = false;
    signed char* planes = nullptr;
    int* rowinfo = nullptr;
    i64* part = nullptr;       // nin 3072: the K slices' partial piles and light facts (sm_plate_product_rows_from)
    int* sfacts = nullptr;
    int* x32 = nullptr;        // sm_plate_product_rows_from: the caller rows' low 32 bits [64][nin]
};

static void plate_free(sm_plate* p) {
    free_plate(p->P);
    free_mfma_plate(p->M);
    hfree(p->planes); hfree(p->rowinfo); hfree(p->part); hfree(p->sfacts); hfree(p->x32);
    delete p;
}

extern "C" int sm_plate_create(const int16_t* w, const int32_t* e, const int64_t* b, int32_t nin, int32_t nout, int32_t tile_cols, sm_plate** out) {
    if (!w || !e || !b || !out) return fail(SM_E_ARG, "sm_plate_create: null argument");
    if (nout <= 0 || nout > (1 << 24)) return fail(SM_E_ARG, "sm_plate_create: nout out of range");
    if (!((nin == 768 && (tile_cols == 0 || tile_cols == 2 || tile_cols == 4 || tile_cols == 8)) ||
          (nin == 3072 && (tile_cols == 0 || tile_cols == 1 || tile_cols == 2))))
        return fail(SM_E_ARG, "sm_plate_create: built for (nin, tile_cols) in (768, 0|2|4|8), (3072, 0|1|2)");
    sm_plate* p = new sm_plate();
    int rc;
    if (tile_cols == 0) {
        p->mfma = true;
        const size_t pb = (size_t)4 * (nin / 64) * 3 * 1024;
        if ((rc = upload_mfma_plate(p->M, w, e, (const i64*)b, nin, nout)) || (rc = dalloc(&p->planes, pb)) ||
            (rc = dalloc(&p->rowinfo, (size_t)64 * 8)) || (rc = dalloc(&p->x32, (size_t)64 * nin)) ||
            (nin == 3072 && ((rc = dalloc(&p->part, (size_t)4 * 64 * (size_t)p->M.ntiles * 16)) ||
                             (rc = dalloc(&p->sfacts, (size_t)4 * 64 * 4))))) {
            plate_free(p);
            return rc;
        }
        if (hipMemset(p->planes, 0, pb) != hipSuccess) { plate_free(p); return fail(SM_E_HIP, "hipMemset planes"); }
    } else if ((rc = upload_plate(p->P, w, e, (const i64*)b, nin, nout, tile_cols))) {
        plate_free(p);
        return rc;
    }
    *out = p;
    return SM_OK;
}
extern "C" int sm_plate_destroy(sm_plate* p) {
    if (p) {
        (void)hipDeviceSynchronize();
        plate_free(p);
    }
    return SM_OK;
}
extern "C" int64_t sm_plate_bytes(const sm_plate* p) {
    if (!p) return 0;
    if (p->mfma) return (int64_t)p->M.ntiles * 16 * p->M.K * 2;
    return (int64_t)p->P.ntiles * p->P.tc * p->P.nin * 2;
}

// the rows' light planes and row facts go to planes / rowinfo (the plate's own, or the static scratch of
// sm_plate_product_rows_noalloc)
// timed: each launch stamped with an event pair (sm_profile_stages); the allocation-free entry point never is, since
// an event pair creates HIP events and records them
template <int RT>
static void rows_product(const sm_plate* p, const int64_t* x16, int32_t rows, int64_t* pile, hipStream_t s,
                         signed char* planes, int* rowinfo, bool timed) {
    const MfmaPlate& P = p->M;
    LightArgs la{};
    la.K = P.K; la.rows = rows; la.X = (const i64*)x16; la.planes = planes; la.rowinfo = rowinfo;
    GemmArgs ga{};
    ga.K = P.K; ga.N = P.N; ga.rows = rows; ga.RT = RT; ga.W = P.W; ga.csum = P.csum; ga.we = P.e; ga.bias = P.b;
    ga.planes = planes; ga.rowinfo = rowinfo; ga.Y = (i64*)pile; ga.ystride = P.N;
    if (P.K == 768) {
        launch(timed, "plate.light", k_light<768, PRO_X16, 192, 1>, dim3(rows), dim3(192), 0, s, la);
        if (P.N > 3072)       // head-shaped plates: the head's kernel (light planes in LDS)
            launch(timed, "plate.head_rows", k_head_rows<RT, EPI_PILE>, dim3(head_rows_grid(P.ntiles)), dim3(256), 0, s, ga);
        else                  // layer-shaped plates: one column tile per block, K split over its four waves
            launch(timed, "plate.gemm", k_gemm<768, 1, 1, EPI_PILE>, dim3(P.ntiles, RT), dim3(256), 0, s, ga);
    } else {
        launch(timed, "plate.light", k_light<3072, PRO_X16, 768, 1>, dim3(rows), dim3(768), 0, s, la);
        launch(timed, "plate.gemm", k_gemm<3072, 1, 1, EPI_PILE>, dim3(P.ntiles, RT), dim3(256), 0, s, ga);
    }
}

extern "C" int sm_plate_product_rows(const sm_plate* p, const int64_t* x16, int32_t rows, int64_t* pile, void* stream) {
    if (!p || !x16 || !pile) return fail(SM_E_ARG, "sm_plate_product_rows: null argument");
    if (!p->mfma) return fail(SM_E_ARG, "sm_plate_product_rows: the plate was made for the GEMV (tile_cols > 0)");
    if (rows < 1 || rows > 64) return fail(SM_E_ARG, "sm_plate_product_rows: rows must be in [1, 64]");
    hipStream_t s = (hipStream_t)stream;
    const int RT = (rows + 15) / 16;
    const bool timed = g_kt.stages;
    if (RT == 1) rows_product<1>(p, x16, rows, pile, s, p->planes, p->rowinfo, timed);
    else if (RT == 2) rows_product<2>(p, x16, rows, pile, s, p->planes, p->rowinfo, timed);
    else if (RT == 3) rows_product<3>(p, x16, rows, pile, s, p->planes, p->rowinfo, timed);
    else rows_product<4>(p, x16, rows, pile, s, p->planes, p->rowinfo, timed);
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// ---------------------------------------------------------------------------------------------------------
// The allocation-free rows product.  Its light planes and row facts live in `scratch`, a file-scope device array
// sized for the largest call (64 rows of a 3072-wide light: 4 row tiles x 48 steps of 64 x 3 planes x 1 KB, then
// 64 x 8 row facts); every GPU this library runs on holds its own copy until the process ends.  Host code never
// passes the array's name to a kernel: on each device the entry point's first call looks its address up (with
// that device current) and keeps it.  Nothing in the scratch needs to start at zero: k_light writes the planes
// and facts of every row it is given before the contraction reads them, the facts of rows past `rows` are read
// through bounded loads (zeros), and a row tile's padding rows feed only their own MFMA output rows, which are
// never stored.  Calls on one GPU share the array, so calls that overlap on one GPU race.
#define SM_NOALLOC_PLANES ((size_t)4 * 48 * 3 * 1024)
#define SM_NOALLOC_BYTES (SM_NOALLOC_PLANES + (size_t)64 * 8 * 4)
static __device__ __align__(256) signed char scratch[SM_NOALLOC_BYTES];
static std::mutex g_scratch_mu;
static signed char* g_scratch_dev[256];              // scratch's address on each device (null: not looked up yet)

static int scratch_on_current_device(signed char** out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 256) return fail(SM_E_ARG, "sm_plate_product_rows_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(SM_E_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_dev[dev] = static_cast<signed char*>(ptr);
    }
    *out = g_scratch_dev[dev];
    return SM_OK;
}

extern "C" int sm_plate_product_rows_noalloc(const sm_plate* p, const int64_t* x16, int32_t rows, int64_t* pile,
                                             void* stream) {
    if (!p || !x16 || !pile) return fail(SM_E_ARG, "sm_plate_product_rows_noalloc: null argument");
    if (!p->mfma) return fail(SM_E_ARG, "sm_plate_product_rows_noalloc: the plate was made for the GEMV (tile_cols > 0)");
    if (rows < 1 || rows > 64) return fail(SM_E_ARG, "sm_plate_product_rows_noalloc: rows must be in [1, 64] (the scratch holds 64)");
    const int RT = (rows + 15) / 16;
    const size_t need = (size_t)RT * (p->M.K / 64) * 3 * 1024;
    if (need > SM_NOALLOC_PLANES) return fail(SM_E_ARG, "sm_plate_product_rows_noalloc: the light planes pass the scratch");
    signed char* base = nullptr;
    int rc;
    if ((rc = scratch_on_current_device(&base))) return rc;
    signed char* planes = base;
    int* rowinfo = reinterpret_cast<int*>(base + SM_NOALLOC_PLANES);
    hipStream_t s = (hipStream_t)stream;
    // untimed whatever sm_profile_stages says: no HIP object is created or recorded on this path
    if (RT == 1) rows_product<1>(p, x16, rows, pile, s, planes, rowinfo, false);
    else if (RT == 2) rows_product<2>(p, x16, rows, pile, s, planes, rowinfo, false);
    else if (RT == 3) rows_product<3>(p, x16, rows, pile, s, planes, rowinfo, false);
    else rows_product<4>(p, x16, rows, pile, s, planes, rowinfo, false);
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

// the machine's proj (nin 768: one block a column tile, the light from 12 OR words a row) and mproj (nin 3072:
// three column tiles a block, four K slices, 192 OR words a row) on the caller's rows
extern "C" int sm_plate_product_rows_from(const sm_plate* p, const int64_t* X, const int64_t* orw, int32_t rows,
                                          int64_t* pile, void* stream) {
    if (!p || !X || !orw || !pile) return fail(SM_E_ARG, "sm_plate_product_rows_from: null argument");
    if (!p->mfma) return fail(SM_E_ARG, "sm_plate_product_rows_from: the plate was made for the GEMV (tile_cols > 0)");
    if (rows < 1 || rows > 64) return fail(SM_E_ARG, "sm_plate_product_rows_from: rows must be in [1, 64]");
    const MfmaPlate& P = p->M;
    if (P.N % 16 != 0 || (P.K == 3072 && P.ntiles % 3 != 0) || (P.K == 768 && P.N > 3072))
        return fail(SM_E_ARG, "sm_plate_product_rows_from: nout must be a multiple of 16 (nin 768, at most 3072) or 48 (nin 3072)");
    hipStream_t s = (hipStream_t)stream;
    const int RT = (rows + 15) / 16;
    GemmArgs ga{};
    ga.K = P.K; ga.N = P.N; ga.rows = rows; ga.RT = RT; ga.W = P.W; ga.csum = P.csum; ga.we = P.e; ga.bias = P.b;
    ga.Y = (i64*)pile; ga.ystride = P.N;
    ga.X = (const i64*)X; ga.xstride = P.K; ga.orw = (const i64*)orw;
    ga.X32 = p->x32;           // the rows' 32-bit copies, read where a row's OR words show that they fit
    {
        const i64 n = (i64)rows * P.K;
        launch(g_kt.stages, "plate.low32", k_low32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const i64*)X, p->x32, n);
    }
    if (P.K == 768) {
        launch(g_kt.stages, "plate.gemm_from", k_gemm<768, 1, 1, EPI_PILE, 12>, dim3(P.ntiles, RT), dim3(256), 0, s, ga);
    } else {
        ga.part = p->part; ga.sfacts = p->sfacts;
        launch(g_kt.stages, "plate.gemm_from", k_gemm<3072, 3, 4, EPI_PART, 192>, dim3(P.ntiles / 3 * 4, RT), dim3(256), 0, s, ga);
        launch(g_kt.stages, "plate.part_piles", k_part_piles<4>, dim3((P.N + 255) / 256, rows), dim3(256), 0, s, ga);
    }
    HIP_TRY(hipGetLastError());
    return SM_OK;
}

extern "C" int sm_plate_product(const sm_plate* p, const int64_t* x16, int64_t* pile, int32_t grid, void* stream) {
    if (!p || !x16 || !pile) return fail(SM_E_ARG, "sm_plate_product: null argument");
    if (p->mfma) return fail(SM_E_ARG, "sm_plate_product: the plate was made for rows (tile_cols == 0)");
    const DevPlate& P = p->P;
    GemvArgs a{};
    a.W = reinterpret_cast<const int4*>(P.W); a.we = P.e; a.bias = P.b; a.sw = P.sw; a.nout = P.nout; a.ntiles = P.ntiles;
    a.X = (const i64*)x16; a.Y = (i64*)pile;
    const int g = grid > 0 ? grid : (P.ntiles + 3) / 4;     // four waves per block, one tile per wave
    hipStream_t s = (hipStream_t)stream;
    if (P.nin == 768 && P.tc == 8) launch(g_kt.stages, "plate.gemv", k_gemv<768, 8, 4, PRO_X16, EPI_PILE, 0>, dim3(g), dim3(256), 0, s, a);
    else if (P.nin == 768 && P.tc == 4) launch(g_kt.stages, "plate.gemv", k_gemv<768, 4, 4, PRO_X16, EPI_PILE, 0>, dim3(g), dim3(256), 0, s, a);
    else if (P.nin == 768 && P.tc == 2) launch(g_kt.stages, "plate.gemv", k_gemv<768, 2, 4, PRO_X16, EPI_PILE, 0>, dim3(g), dim3(256), 0, s, a);
    else if (P.nin == 3072 && P.tc == 1) launch(g_kt.stages, "plate.gemv", k_gemv<3072, 1, 4, PRO_X16, EPI_PILE, 0>, dim3(g), dim3(256), 0, s, a);
    else launch(g_kt.stages, "plate.gemv", k_gemv<3072, 2, 4, PRO_X16, EPI_PILE, 0>, dim3(g), dim3(256), 0, s, a);
    HIP_TRY(hipGetLastError());
    return SM_OK;
}
