// pcdevice.hip -- C ABI of libpcdevice_hip (declared in include/pcdevice.h).
//
// Host side of the MI355X relaxation: the device runtime calls the reference
// binds through P/Invoke (PredictiveCoding.Device/Interop/*.cs), a pooled
// allocator (Allocators/CudaAllocator.cs), streams and events
// (Streams/CudaStreamManager.cs), row-major GEMMs (Gemm/CudaGemmProvider.cs)
// and the batched relaxation itself (BatchedPcForward.cs) with its ragged,
// early-exit variant (Network.cs:760-907 applied per request).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/pcdevice.h"
#include "aux_kernels.hpp"
#include "phase_launch.hpp"

using namespace pcd;

namespace {

// ------------------------------------------------------------------ errors

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return PCD_SUCCESS;
    int st = PCD_HIP_ERROR;
    if (e == hipErrorNoDevice) st = PCD_NO_DEVICE;
    else if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) st = PCD_OUT_OF_MEMORY;
    else if (e == hipErrorInvalidValue || e == hipErrorInvalidDevicePointer || e == hipErrorInvalidDevice)
        st = PCD_INVALID_VALUE;
    else if (e == hipErrorNotSupported) st = PCD_NOT_SUPPORTED;
    return fail(st, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(call)                                    \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return from_hip(e_, #call); \
    } while (0)

// HIP refuses an operation on the legacy (null) stream, such as a synchronous
// hipMemcpy, hipMemset or hipDeviceSynchronize, while any stream of the
// process is capturing a graph, whatever the capture mode, and invalidates
// that capture too (hipErrorStreamCaptureImplicit, then
// hipErrorStreamCaptureInvalidated for the capturing thread).  The library's
// own captures (get_plan) and its legacy-stream calls therefore exclude each
// other: two callers on two threads, one recording a settling's graph and one
// copying its inputs, both succeed.  Nothing else is locked while this is held
// except the pool's mutex inside a capture, and no holder of the pool's mutex
// waits for this one.
std::mutex& legacy_stream_mu() {
    static std::mutex mu;
    return mu;
}
hipError_t sync_memcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    std::lock_guard<std::mutex> g(legacy_stream_mu());
    return hipMemcpy(dst, src, bytes, kind);
}
hipError_t sync_memset(void* dst, int value, size_t bytes) {
    std::lock_guard<std::mutex> g(legacy_stream_mu());
    return hipMemset(dst, value, bytes);
}
hipError_t device_sync() {
    std::lock_guard<std::mutex> g(legacy_stream_mu());
    return hipDeviceSynchronize();
}

inline size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// --------------------------------------------------------------- allocator

// Power-of-two buckets of at most 32 cached blocks per (device, stream), as
// CudaAllocator does (CudaAllocator.cs:32-59,98-103).  A block freed on a
// stream is handed out again only on that stream, so stream order alone keeps
// a reused block from racing with work still queued on it.
struct Pool {
    std::mutex mu;
    struct Key {
        int dev;
        void* stream;
        int bucket;
        bool operator<(const Key& o) const {
            if (dev != o.dev) return dev < o.dev;
            if (stream != o.stream) return stream < o.stream;
            return bucket < o.bucket;
        }
    };
    std::map<Key, std::vector<void*>> free_blocks;
    std::unordered_map<void*, std::pair<int, int>> live;  // ptr -> (device, bucket)
    std::unordered_map<void*, bool> synchronous;          // blocks from the hipMalloc fallback (freed with hipFree)
    std::map<int, std::vector<void*>> host_free;          // bucket -> pinned blocks
    std::unordered_map<void*, int> host_live;
    static constexpr size_t kMaxCached = 32;
};
Pool& pool() {
    static Pool* p = new Pool();  // leaked on purpose: outlives static destructors
    return *p;
}

int bucket_of(size_t bytes) {
    int b = 8;  // 256 B minimum
    while (((size_t)1 << b) < bytes) ++b;
    return b;
}

int pool_alloc(void** out, size_t bytes, hipStream_t stream) {
    if (!out) return fail(PCD_INVALID_VALUE, "pcd_malloc_async: null out pointer");
    *out = nullptr;
    if (bytes == 0) return PCD_SUCCESS;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    int b = bucket_of(bytes);
    Pool& P = pool();
    {
        std::lock_guard<std::mutex> g(P.mu);
        auto it = P.free_blocks.find({dev, (void*)stream, b});
        if (it != P.free_blocks.end() && !it->second.empty()) {
            *out = it->second.back();
            it->second.pop_back();
            P.live[*out] = {dev, b};
            return PCD_SUCCESS;
        }
    }
    void* p = nullptr;
    bool fallback = false;
    hipError_t e = hipMallocAsync(&p, (size_t)1 << b, stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        e = hipMalloc(&p, (size_t)1 << b);  // CudaAllocator.cs:43-44 fallback
        fallback = true;
    }
    if (e != hipSuccess) return from_hip(e, "pcd_malloc_async");
    std::lock_guard<std::mutex> g(P.mu);
    P.live[p] = {dev, b};
    if (fallback) P.synchronous[p] = true;
    *out = p;
    return PCD_SUCCESS;
}

int pool_free(void* ptr, hipStream_t stream) {
    if (!ptr) return PCD_SUCCESS;
    Pool& P = pool();
    std::lock_guard<std::mutex> g(P.mu);
    auto it = P.live.find(ptr);
    if (it == P.live.end()) return fail(PCD_INVALID_VALUE, "pcd_free_async: pointer not from pcd_malloc_async");
    auto [dev, b] = it->second;
    P.live.erase(it);
    auto& v = P.free_blocks[{dev, (void*)stream, b}];
    if (v.size() < Pool::kMaxCached) {
        v.push_back(ptr);
        return PCD_SUCCESS;
    }
    // A block of the stream-ordered allocator goes back to it in stream order;
    // one from the synchronous fallback must not be handed to hipFreeAsync.
    auto fb = P.synchronous.find(ptr);
    if (fb != P.synchronous.end()) {
        P.synchronous.erase(fb);
        HIP_TRY(hipStreamSynchronize(stream));   // the stream's queued work may still use it
        HIP_TRY(hipFree(ptr));
        return PCD_SUCCESS;
    }
    HIP_TRY(hipFreeAsync(ptr, stream));
    return PCD_SUCCESS;
}

// ------------------------------------------------------------------ launch

template <typename OP, int BM, int BN>
int launch_tile(int epi, const ProblemSet& set, const PhaseArgs& args, int grid, hipStream_t s) {
    return from_hip(launch_phase_tile<OP, BM, BN>(epi, set, args, grid, s), "phase_kernel launch");
}

// GEMM tile shapes compiled into the library (rows x columns of the output).
// wd: the direct-weight 64 x 128 tile of the 16-bit settlings, whose weight
// operand is the model's fragment-major copy (never chosen by the caller).
struct Tile {
    int m, n;
    bool wd = false;
};
bool same_tile(Tile a, Tile b) { return a.m == b.m && a.n == b.n && a.wd == b.wd; }
bool tile_supported(Tile t) {
    return (t.m == 32 && t.n == 32) || (t.m == 64 && (t.n == 64 || t.n == 128 || t.n == 256)) ||
           (t.m == 128 && t.n == 128) || (t.m == 256 && t.n == 128) || (t.m == 256 && t.n == 256);
}

template <typename OP>
int launch_op(Tile tile, int epi, const ProblemSet& set, const PhaseArgs& args, int grid, hipStream_t s) {
    if (tile.wd) {
        if constexpr (std::is_same<OP, float>::value) return fail(PCD_INVALID_VALUE, "direct-weight tile on fp32");
        else return from_hip(launch_phase_tile<OP, 64, 128, true>(epi, set, args, grid, s), "phase_kernel launch");
    }
    if (tile.m == 32 && tile.n == 32) return launch_tile<OP, 32, 32>(epi, set, args, grid, s);
    if (tile.m == 64 && tile.n == 64) return launch_tile<OP, 64, 64>(epi, set, args, grid, s);
    if (tile.m == 64 && tile.n == 128) return launch_tile<OP, 64, 128>(epi, set, args, grid, s);
    if (tile.m == 64 && tile.n == 256) return launch_tile<OP, 64, 256>(epi, set, args, grid, s);
    if (tile.m == 128 && tile.n == 128) return launch_tile<OP, 128, 128>(epi, set, args, grid, s);
    if (tile.m == 256 && tile.n == 128) return launch_tile<OP, 256, 128>(epi, set, args, grid, s);
    if (tile.m == 256 && tile.n == 256) return launch_tile<OP, 256, 256>(epi, set, args, grid, s);
    return fail(PCD_INVALID_VALUE, "unsupported tile %d x %d", tile.m, tile.n);
}

// Workgroups of a phase launch: 8 x the most tiles any XCD runs (the kernel
// deals the tiles over the XCDs with xcd_share, per problem or in one run).
int phase_grid(const ProblemSet& set, int order) {
    int most = 0, total = 0;
    for (int i = 0; i < set.n; ++i) total += set.p[i].tiles;
    for (int x = 0; x < kXcds; ++x) {
        int sum = 0, lo, cnt;
        if (order == TILE_INTERLEAVED) {
            for (int i = 0; i < set.n; ++i) {
                xcd_share(set.p[i].tiles, x, lo, cnt);
                sum += cnt;
            }
        } else {
            xcd_share(total, x, lo, cnt);
            sum = cnt;
        }
        most = std::max(most, sum);
    }
    return most * kXcds;
}

int launch_phase(int dtype, Tile tile, int epi, const ProblemSet& set, const PhaseArgs& args, hipStream_t s) {
    const int grid = phase_grid(set, args.tile_order);
    if (grid == 0) return PCD_SUCCESS;
    switch (dtype) {
    case PCD_F32: return launch_op<float>(tile, epi, set, args, grid, s);
    case PCD_BF16: return launch_op<bf16_t>(tile, epi, set, args, grid, s);
    case PCD_F16: return launch_op<f16_t>(tile, epi, set, args, grid, s);
    default: return fail(PCD_INVALID_VALUE, "unknown dtype %d", dtype);
    }
}

int launch_zero(void* p, size_t bytes, hipStream_t s) {
    size_t units = bytes / 16;
    if (units == 0) return PCD_SUCCESS;
    int grid = (int)std::min<size_t>((units + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(256), 0, s, (u32x4*)p, units);
    return from_hip(hipGetLastError(), "zero_kernel launch");
}

// Buffers to zero, gathered and cleared by one zero_segs_kernel launch per
// kZeroSegs of them.
struct ZeroBatch {
    ZeroSegs z{};
    size_t most = 0;   // units of the largest buffer gathered
    int add(void* p, size_t bytes, hipStream_t s) {
        const size_t units = bytes / 16;
        if (units == 0) return PCD_SUCCESS;
        if (z.count == kZeroSegs)
            if (int st = flush(s)) return st;
        z.p[z.count] = (u32x4*)p;
        z.n[z.count++] = units;
        most = std::max(most, units);
        return PCD_SUCCESS;
    }
    int flush(hipStream_t s) {
        if (z.count == 0) return PCD_SUCCESS;
        const int grid = (int)std::min<size_t>((most + 255) / 256, 4096);
        hipLaunchKernelGGL(zero_segs_kernel, dim3(grid), dim3(256), 0, s, z);
        z.count = 0;
        most = 0;
        return from_hip(hipGetLastError(), "zero_segs_kernel launch");
    }
};

inline int op_bytes(int dtype) { return dtype == PCD_F32 ? 4 : 2; }

// --------------------------------------------------------------- PC model

constexpr int kFeatPad = 64;    // feature dims padded to the deepest LDS stage (64 elements)
constexpr int kRowPad = 256;    // row dims padded to the widest tile
constexpr int kMinTileM = 32;   // rows of the shortest tile
// Learning steps of at most this many rows update the weights with
// hebbian_small_kernel (K = rows on the VALU, every layer in one launch)
// instead of transposing D and M for a grouped MFMA GEMM and refreshing the
// operand copies layer by layer (measured faster up to 512 rows on c1's and
// c2's networks, slower at 1024 on c2's).
constexpr int kHebbValuRows = 512;
// K stagger of the settling phases and GEMMs with 16-bit operands: spreads
// the tiles that share operand rows over 16 stage offsets (measured on 6 x 4096
// and 12 x 8192 bf16 networks: 7-10% faster than no stagger, and better than 4
// or 8 offsets).  fp32 gained nothing measurable and keeps it off, which also
// keeps every row's result independent of the other rows in the batch.
// K stagger of a 16-bit GEMM sweeping nk stages when the option is left
// automatic: a quarter of the stages (measured best at nk = 64 and 128: c3's
// and c5's settling phases, the 8192^3 provider GEMM); half of them when the
// rows fit one row tile, where no two tiles share weight rows and the stride
// only spreads the weight streams (c5's network at 64 rows), within
// [2, kMaxKStagger].
constexpr int kKStaggerAuto = -1;
int auto_k_stagger(int nk, bool one_row_tile = false);
constexpr int kMaxKStagger = 64;
// Fewest K stages a split-K range runs: a range also pays its partial tile's
// store, the count and (last range) the reduction, a few microseconds.
#ifndef PCD_SPLIT_MIN_STAGES
#define PCD_SPLIT_MIN_STAGES 12
#endif
constexpr int kSplitMinStages = PCD_SPLIT_MIN_STAGES;
// The same on the K-shared 32 x 32 tile, whose ranges publish and sum a
// quarter of a block per wave (784-256-256-10 at a batch of 64: 4 beats 12
// by 6%, 2 loses 5%).
constexpr int kSplitMinStagesKsw = 4;
// Persistent settling buffer: the grid barrier's arrival count and give-up flag.
constexpr size_t kPersistBytes = 256;
constexpr int kPersistSpinDefault = 1 << 22;   // about a second of polls (each a device-scope load and a sleep)

struct Plan;

// Per (model, stream) device buffers for batches up to `cap` rows.
struct Workspace {
    hipStream_t stream = nullptr;
    int cap = 0;                       // rows, multiple of kRowPad
    std::vector<float*> M;             // [L] fp32 states (M[0] = clamped input)
    std::vector<void*> S;              // [L] operand-type state copies (16-bit dtypes only)
    std::vector<void*> D;              // [L] D_l, l >= 1, operand type [cap x P_{l-1}]
    std::vector<float*> E;             // [L] X_l = M_l - eta (E_l + lambda sign M_l), 1 <= l <= L-2, fp32 [cap x P_l]
    float* energy_part = nullptr;      // [slots x cap]
    int slots_cap = 0;
    float* split_part = nullptr;       // split-K partial tiles, split_part_tiles() x 128 x 128 fp32
    int* split_count = nullptr;        // split-K finished-range counters, zero between launches
    int* act_tm = nullptr;             // ragged: row tiles still running at the current step [cap / kMinTileM]
    int* act_count = nullptr;          // ragged: their number
    void* persist = nullptr;           // persistent settling: the grid barrier's arrival count and give-up flag
    void* rg_tables = nullptr;         // ragged: per-call tables (see pcd_pc_relax_ragged), sized for cap rows
    hipStream_t capture = nullptr;     // private stream used for graph capture
    std::vector<std::unique_ptr<Plan>> plans;
    std::vector<void*> owned;          // every hipMalloc'ed buffer
};

struct Plan {
    int batch = 0, steps = 0, want_energy = 0, clamp_top = 0, keep_hidden = 0;
    Tile tile{0, 0};
    // ragged loops (requests > 0): their tables live in the workspace at
    // offsets fixed by (batch, requests), so these complete the key
    int requests = 0, exit_rule = 0;
    float exit_thr = 0.f;
    float* energy_out = nullptr;       // [steps x batch]
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    uint64_t last_use = 0;

    Plan() = default;
    Plan(const Plan&) = delete;
    Plan& operator=(const Plan&) = delete;
    // The owner makes sure no launch of the graph is still queued (it
    // synchronises the stream the plan was launched on first).
    ~Plan() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (energy_out) (void)hipFree(energy_out);
    }
};

}  // namespace

struct pcd_model {
    int device = 0;
    int cus = 256;                      // compute units of the device
    int L = 0;
    std::vector<int> s, P;              // sizes, padded sizes (the GEMMs' K and every buffer's row pitch)
    int act = 0, ffg = 0, dtype = 0;
    float eta = 0.f, act_reg = 0.f;
    std::vector<float> prec;
    std::vector<void*> W, WT;           // [L] operand type; W[l] is [R(s_{l-1}) x P_l], WT[l] [R(s_l) x P_{l-1}]
    std::vector<float*> W32;            // [L] fp32 master weights of 16-bit models, laid out as W[l]
    // [L] fragment-major copies of W[l] and WT[l] (frag_pack_kernel), kept for
    // 16-bit models whose small-batch settlings take the direct-weight tile
    // (direct_eligible); refreshed wherever W[l] and WT[l] change
    std::vector<void*> Wpk, WTpk;
    std::vector<float*> bias;           // [L] fp32 [P_{l-1}]
    std::mutex mu;
    std::vector<std::unique_ptr<Workspace>> ws;
    // options
    int use_graph = 1, tile_m = 0, tile_n = 0, profile = 0, tile_order = TILE_INTERLEAVED, split_k = 1;
    int persistent = 0;                 // fixed-step fp32 settlings of few tiles as one persistent launch (opt-in)
    int split_min = 0;                  // fewest K stages of a split-K range in the settling phases (0: by tile)
    int persist_spin = kPersistSpinDefault;
    int persist_grid = 0;               // workgroups of the persistent launch (0: automatic)
    int k_stagger = 0;                  // settling phases: kKStaggerAuto (16-bit default), 0 off, or a fixed value
    int ragged_tiles = 1;               // ragged phases deal only the row tiles still running
    int ragged_order = 1;               // ragged requests settle in decreasing step budget (0: caller's order)
    int direct = 1;                     // direct-weight tile: 0 never, 1 where direct_eligible, 2 every batch <= 64 rows
    int nt_store = -1;                  // settling epilogues' stores non-temporal: -1 automatic (see relax_args), 0, 1
    int nt_load = -1;                   // settling epilogues' fp32 state loads non-temporal: -1 automatic, 0, 1
    float prof_err_ms = 0.f, prof_upd_ms = 0.f;
    int prof_launches = 0;
    uint64_t clock = 0;
};

namespace {

// Callers have synchronised the workspace's stream (or the device).
void free_workspace(Workspace& w) {
    w.plans.clear();
    for (void* p : w.owned) (void)hipFree(p);
    w.owned.clear();
    w.rg_tables = nullptr;
    if (w.capture) (void)hipStreamDestroy(w.capture);
    w.capture = nullptr;
}

int dev_alloc_zero(std::vector<void*>& owned, void** out, size_t bytes) {
    *out = nullptr;
    if (bytes == 0) return PCD_SUCCESS;
    HIP_TRY(hipMalloc(out, bytes));
    owned.push_back(*out);
    HIP_TRY(sync_memset(*out, 0, bytes));
    return PCD_SUCCESS;
}

// Fragment-major copies of layer l's operand-type weights (W[l] and WT[l]),
// for models that keep them; enqueued on s after whatever wrote W[l] and WT[l].
int repack_direct(pcd_model* m, int l, hipStream_t s) {
    if (m->Wpk.empty() || !m->Wpk[l]) return PCD_SUCCESS;
    const int Rlo = (int)round_up(m->s[l - 1], kRowPad), Rsz = (int)round_up(m->s[l], kRowPad);
    const int g1 = (int)std::min<size_t>(((size_t)Rlo * m->P[l] / 8 + 255) / 256, 8192);
    const int g2 = (int)std::min<size_t>(((size_t)Rsz * m->P[l - 1] / 8 + 255) / 256, 8192);
    hipLaunchKernelGGL(frag_pack_kernel, dim3(g1), dim3(256), 0, s, (const u32x4*)m->W[l], m->P[l], Rlo, m->P[l],
                       (u32x4*)m->Wpk[l]);
    hipLaunchKernelGGL(frag_pack_kernel, dim3(g2), dim3(256), 0, s, (const u32x4*)m->WT[l], m->P[l - 1], Rsz,
                       m->P[l - 1], (u32x4*)m->WTpk[l]);
    return from_hip(hipGetLastError(), "frag_pack_kernel launch");
}

// Allocates and fills the fragment-major weight copies of a 16-bit model
// that does not keep them (the option that forces the direct-weight tile).
int alloc_direct(pcd_model* m) {
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(device_sync());   // the weights may still be written by queued work
    std::vector<void*> owned;
    std::vector<void*> wpk(m->L, nullptr), wtpk(m->L, nullptr);
    int st = PCD_SUCCESS;
    for (int l = 1; l < m->L && !st; ++l) {
        const size_t rlo = round_up(m->s[l - 1], kRowPad), rsz = round_up(m->s[l], kRowPad);
        st = dev_alloc_zero(owned, &wpk[l], rlo * m->P[l] * 2);
        if (!st) st = dev_alloc_zero(owned, &wtpk[l], rsz * m->P[l - 1] * 2);
    }
    if (!st) {
        m->Wpk = wpk;
        m->WTpk = wtpk;
        for (int l = 1; l < m->L && !st; ++l) st = repack_direct(m, l, 0);
        if (!st) st = from_hip(device_sync(), "direct-weight copies");
        if (!st) return PCD_SUCCESS;
        m->Wpk.clear();
        m->WTpk.clear();
    }
    for (void* p : owned) (void)hipFree(p);
    return st;
}

// Tiles of one error phase at `batch` rows.
long error_phase_tiles(const pcd_model* m, int batch, Tile t) {
    long tiles = 0;
    const long tm = (batch + t.m - 1) / t.m;
    for (int l = 1; l < m->L; ++l) tiles += tm * ((m->s[l - 1] + t.n - 1) / t.n);
    return tiles;
}

// The largest tile that still gives every CU at least two workgroups per
// phase (a phase with fewer tiles leaves SIMDs idle: 64 x 64 beats 128 x 128
// by 8% on the 1024-wide fp32 configuration).  256 x 256 only for 16-bit
// operands with every layer at least 1024 wide.  A settling whose error
// phase has fewer 64 x 64 tiles than the GPU has CUs takes the K-shared
// 32 x 32 tile: its phases are bound by one tile's K sweep, which that tile
// runs four times as fast, and by the epilogue, which it splits over the
// waves (784-256-256-10 at a batch of 64: fp32 +88%, bf16 +34%), unless the
// fp32 persistent form, built on 64 x 64, is asked for.
Tile choose_tile(const pcd_model* m, int batch) {
    if (m->tile_m > 0) return Tile{m->tile_m, m->tile_n};
    const bool have_direct = m->direct && !m->Wpk.empty() && m->Wpk[1];
    if (m->direct == 2 && have_direct && batch <= 64) return Tile{64, 128, true};   // forced (option)
    if (!(m->dtype == PCD_F32 && m->persistent) && error_phase_tiles(m, batch, Tile{64, 64}) < m->cus)
        return Tile{32, 32};
    // A batch that fits one 64-row tile: any taller tile is mostly padding rows
    // (its MFMAs and its state loads wasted), and the phases stream weights,
    // which the direct-weight tile streams fastest (c5's network at 64 rows:
    // the weights at 5.8 TB/s in its main loop against 5.0 for 64 x 64).
    if (batch <= 64) return have_direct ? Tile{64, 128, true} : Tile{64, 64};
    const long want = 2L * m->cus;
    if (m->dtype != PCD_F32) {
        bool wide = true;
        for (int l = 0; l < m->L; ++l) wide = wide && m->s[l] >= 1024;
        if (wide && error_phase_tiles(m, batch, Tile{256, 256}) >= want) return Tile{256, 256};
    }
    if (error_phase_tiles(m, batch, Tile{128, 128}) >= want) return Tile{128, 128};
    return Tile{64, 64};
}

// Whether a 16-bit model keeps fragment-major weight copies for the
// direct-weight tile: its batches of up to 64 rows run 64 x 64 tiles otherwise
// (not the K-shared 32 x 32), and its error phase has at least one
// direct-weight tile per CU.
bool direct_eligible(const pcd_model* m) {
    return m->dtype != PCD_F32 && error_phase_tiles(m, 64, Tile{64, 64}) >= m->cus &&
           error_phase_tiles(m, 64, Tile{64, 128, true}) >= m->cus;
}

// Energy partial slots a tile column owns: one per wave column of the tile.
int slots_per_tile_n(Tile t) {
    if (t.wd) return energy_slots_per_tile_n<64, 128, true>();
    if (t.m == 32 && t.n == 32) return energy_slots_per_tile_n<32, 32>();
    if (t.m == 256 && t.n == 256) return energy_slots_per_tile_n<256, 256>();
    if (t.m == 256 && t.n == 128) return energy_slots_per_tile_n<256, 128>();
    if (t.m == 128 && t.n == 128) return energy_slots_per_tile_n<128, 128>();
    if (t.m == 64 && t.n == 128) return energy_slots_per_tile_n<64, 128>();
    if (t.m == 64 && t.n == 256) return energy_slots_per_tile_n<64, 256>();
    return energy_slots_per_tile_n<64, 64>();
}

// Energy partial slots of one step with `tile`.
int energy_slots(const pcd_model* m, Tile tile) {
    int slots = 0;
    for (int l = 1; l < m->L; ++l) slots += (int)((m->s[l - 1] + tile.n - 1) / tile.n) * slots_per_tile_n(tile);
    return slots;
}

// The most slots any supported tile needs (sizes the workspace once).
int max_energy_slots(const pcd_model* m) {
    const Tile tiles[] = {{32, 32}, {64, 64}, {64, 128}, {64, 256}, {128, 128}, {256, 128}, {256, 256}, {64, 128, true}};
    int slots = 0;
    for (Tile t : tiles) slots = std::max(slots, energy_slots(m, t));
    return slots;
}

// Launches pack_kernel over the [prow x pcol] destination: 64 x 64 tiles, a
// column of tiles per workgroup column, about 4096 workgroups in all (each
// walks down several tile rows when the matrix is large).
template <typename OP>
void pack_op(hipStream_t s, const void* src, int src_is_f32, int rows, int cols, int trans, void* dst, int prow,
             int pcol, int ldd) {
    const int tiles_x = (pcol + 63) / 64, tiles_y = (prow + 63) / 64;
    const int gy = std::max(1, std::min({tiles_y, 65535, (4096 + tiles_x - 1) / tiles_x}));
    const dim3 grid((unsigned)tiles_x, (unsigned)gy);
    hipLaunchKernelGGL(pack_kernel<OP>, grid, dim3(256), 0, s, src, src_is_f32, rows, cols, trans, dst, prow, pcol,
                       ldd);
}

// Split-K.  A phase whose output tiles leave CUs idle (at most half as many
// tiles as CUs, tiles of at most 128 x 128) cuts each tile's K into up to
// cus / tiles (<= kMaxSplit) ranges of at least kSplitMinStages stages; the partial tiles
// go to workspace scratch and the range that finishes last reduces them and
// runs the epilogue.  The scratch holds `cus` partial tiles of 128 x 128, or
// 4 and 16 times as many of 64 x 64 and 32 x 32, and a counter per split tile
// (at most half the partial tiles: a split tile has two ranges or more);
// assign_split decides how much of it a phase may use.
int split_part_tiles(const pcd_model* m) { return std::max(m->cus, 1); }
constexpr int kSplitCountsPerPart = 8;   // counters per 128 x 128 of scratch: the 32 x 32 tile's 16 / 2
// Bytes of the split-K counters, whole 16-byte units so a zero kernel covers them.
size_t split_count_bytes(int part_tiles) { return round_up((size_t)part_tiles * kSplitCountsPerPart * 4, 16); }
size_t split_count_bytes(const pcd_model* m) { return split_count_bytes(split_part_tiles(m)); }


int split_factor(int cus, int split_k, long tiles, Tile tile) {
    if (!split_k || tile.wd || tile.m * tile.n > 128 * 128 || tiles < 1 || tiles * 2 > cus) return 1;
    return (int)std::min<long>(kMaxSplit, cus / tiles);
}

// K elements of one LDS stage of `tile` for an operand type.
template <int OPB> int stage_rb(Tile t) {
    if (t.m == 32 && t.n == 32) return TileCfg<32, 32, OPB>::RB;
    if (t.m == 64 && t.n == 64) return TileCfg<64, 64, OPB>::RB;
    if (t.m == 64 && t.n == 128) return TileCfg<64, 128, OPB>::RB;
    if (t.m == 64 && t.n == 256) return TileCfg<64, 256, OPB>::RB;
    if (t.m == 128 && t.n == 128) return TileCfg<128, 128, OPB>::RB;
    if (t.m == 256 && t.n == 128) return TileCfg<256, 128, OPB>::RB;
    return TileCfg<256, 256, OPB>::RB;
}

int stage_k(int dtype, Tile tile) {
    const int rb = dtype == PCD_F32 ? stage_rb<4>(tile) : stage_rb<2>(tile);
    return rb / op_bytes(dtype);
}

// The split-K plan of a phase or a GEMM: every problem's split factor and its
// share of the partial-tile scratch (`part`, room for `budget` partial tiles of
// 128 x 128, that is budget * 128 * 128 / (BM * BN) of a BM x BN tile) and of
// the counters (`count`, budget * kSplitCountsPerPart of them).
struct SplitScratch {
    float* part = nullptr;
    int* count = nullptr;
    long budget = 0;
};

// Gives every problem of a phase its split factor and its share of the scratch.
// Besides the few-tiles split of the whole phase, a problem whose eighth (one
// XCD's share) has fewer tiles than the XCD has CUs is split to about one unit
// per CU: its tiles would otherwise give a part of the CUs one more whole tile
// than the rest (c2's update phase: 8 tiles of the 256-wide layer per XCD of 32
// CUs next to 3 x 32 full tiles).  Splitting stops where the scratch is spent.
void assign_split(int cus, int split_k, int dtype, Tile tile, const SplitScratch& sc, std::vector<ProblemSet>& sets,
                  int min_stages = kSplitMinStages) {
    long tiles = 0;
    for (auto& ps : sets)
        for (int i = 0; i < ps.n; ++i) tiles += (long)ps.p[i].tiles_m * ps.p[i].tiles_n;
    const int f = split_factor(cus, split_k, tiles, tile);
    const int per_xcd = std::max(1, cus / kXcds);
    const bool small_tile = tile.m * tile.n <= 128 * 128;
    auto wanted = [&](const Problem& p) {
        const int t = p.tiles_m * p.tiles_n;
        const int share = (t + kXcds - 1) / kXcds;
        const int fb = (split_k && small_tile && !tile.wd && share < per_xcd) ? per_xcd / share : 1;
        return std::max(1, std::min({std::max(f, fb), kMaxSplit, p.K / stage_k(dtype, tile) / min_stages}));
    };
    // All or nothing: a phase whose splits do not all fit the scratch splits
    // none of its problems (splitting only the first ones would leave those
    // slower than the rest: c5s's phases, 11 problems of 16 tiles per XCD).
    long need = 0, need_counters = 0;
    for (auto& ps : sets)
        for (int i = 0; i < ps.n; ++i) {
            const int ks = wanted(ps.p[i]);
            if (ks > 1) {
                need += (long)ps.p[i].tiles_m * ps.p[i].tiles_n * ks;
                need_counters += (long)ps.p[i].tiles_m * ps.p[i].tiles_n;
            }
        }
    // A few-tiles phase (f > 1: half the CUs or more idle unsplit) gets the
    // scratch counted in partial tiles of its own size: the 32 x 32 tile's
    // phases need many (3072-512-128-10's update splits 32 tiles eight ways
    // and 8 tiles four ways, 288 partial tiles of 32 x 32).  Balance splits of
    // phases with more tiles keep the budget of `sc.budget` partial tiles of
    // any size: given more, they made 2048 x 6 bf16 at 128 rows (64 x 64
    // tiles, each CU holding its share at once) 78% slower.
    const long budget = f > 1 ? sc.budget * (128L * 128) / ((long)tile.m * tile.n) : sc.budget;
    const bool fits = need <= budget && need_counters <= sc.budget * kSplitCountsPerPart;
    long units = 0, counters = 0;
    for (auto& ps : sets)
        for (int i = 0; i < ps.n; ++i) {
            Problem& p = ps.p[i];
            const int t = p.tiles_m * p.tiles_n;
            const int ks = fits ? wanted(p) : 1;
            p.ksplit = ks;
            p.tiles = t * ks;
            if (ks > 1) {
                p.part = sc.part + units * (long)tile.m * tile.n;
                p.count = sc.count + counters;
                units += (long)t * ks;
                counters += t;
            }
        }
}


int ensure_workspace(pcd_model* m, hipStream_t stream, int rows, Workspace** out) {
    Workspace* w = nullptr;
    for (auto& x : m->ws)
        if (x->stream == stream) w = x.get();
    if (!w) {
        m->ws.emplace_back(new Workspace());
        w = m->ws.back().get();
        w->stream = stream;
    }
    int need = (int)round_up((size_t)std::max(rows, 1), kRowPad);
    int slots = max_energy_slots(m);
    if (w->cap >= need && w->slots_cap >= slots) {
        *out = w;
        return PCD_SUCCESS;
    }
    HIP_TRY(hipStreamSynchronize(stream));
    free_workspace(*w);
    const int L = m->L, ob = op_bytes(m->dtype);
    w->cap = need;
    w->M.assign(L, nullptr);
    w->S.assign(L, nullptr);
    w->D.assign(L, nullptr);
    w->E.assign(L, nullptr);
    int st;
    for (int l = 0; l < L; ++l) {
        if ((st = dev_alloc_zero(w->owned, (void**)&w->M[l], (size_t)need * m->P[l] * 4))) return st;
        if (l >= 1 && m->dtype != PCD_F32)
            if ((st = dev_alloc_zero(w->owned, &w->S[l], (size_t)need * m->P[l] * ob))) return st;
        if (l >= 1)
            if ((st = dev_alloc_zero(w->owned, &w->D[l], (size_t)need * m->P[l - 1] * ob))) return st;
        if (l >= 1 && l <= L - 2)
            if ((st = dev_alloc_zero(w->owned, (void**)&w->E[l], (size_t)need * m->P[l] * 4))) return st;
    }
    w->slots_cap = slots;
    if ((st = dev_alloc_zero(w->owned, (void**)&w->energy_part, (size_t)slots * need * 4))) return st;
    if ((st = dev_alloc_zero(w->owned, (void**)&w->split_part, (size_t)split_part_tiles(m) * 128 * 128 * 4)))
        return st;
    if ((st = dev_alloc_zero(w->owned, (void**)&w->split_count, split_count_bytes(m)))) return st;
    if ((st = dev_alloc_zero(w->owned, (void**)&w->act_tm, (size_t)(need / kMinTileM) * 4))) return st;
    if ((st = dev_alloc_zero(w->owned, (void**)&w->act_count, 4))) return st;
    if ((st = dev_alloc_zero(w->owned, &w->persist, kPersistBytes))) return st;
    HIP_TRY(hipStreamCreateWithFlags(&w->capture, hipStreamNonBlocking));
    *out = w;
    return PCD_SUCCESS;
}

// Operand of the error-phase GEMM for layer l: the fp32 state itself, or its
// 16-bit copy.
const void* state_operand(const pcd_model* m, const Workspace* w, int l) {
    return m->dtype == PCD_F32 ? (const void*)w->M[l] : w->S[l];
}

// Problem sets of the two phases for a batch; problems beyond kMaxProblems
// spill into further sets (still one phase: the problems are independent).
void build_phase_sets(const pcd_model* m, const Workspace* w, int batch, Tile tile, int clamp_top,
                      std::vector<ProblemSet>& err, std::vector<ProblemSet>& upd, int* nslots) {
    err.clear();
    upd.clear();
    const int L = m->L;
    const int tm = (batch + tile.m - 1) / tile.m;
    int slot = 0;
    // Error phase, layers in ascending order: the energy slots then follow
    // e_0, e_1, ... in the order the reference forms the layer errors
    // (BatchedPcForward.cs:100-107), and the order measured 1% faster than
    // descending on c5s (0.5% on c1).
    for (int l = 1; l < L; ++l) {
        if (err.empty() || err.back().n == kMaxProblems) { err.emplace_back(); err.back().n = 0; }
        ProblemSet& ps = err.back();
        Problem& p = ps.p[ps.n++];
        std::memset(&p, 0, sizeof p);
        p.A = state_operand(m, w, l);
        p.lda = m->P[l];
        p.B = tile.wd ? m->Wpk[l] : m->W[l];
        p.ldb = m->P[l];
        p.M = batch;
        p.N = m->s[l - 1];
        p.K = m->P[l];
        p.tiles_m = tm;
        p.tiles_n = (p.N + tile.n - 1) / tile.n;
        p.tiles = p.tiles_m * p.tiles_n;
        p.ldo = m->P[l - 1];
        p.bias = m->bias[l];
        p.mlow = w->M[l - 1];
        p.eout = l - 1 >= 1 ? w->E[l - 1] : nullptr;
        p.dout = w->D[l];
        p.prec = m->prec[l - 1];
        p.slot_base = slot;
        slot += p.tiles_n * slots_per_tile_n(tile);
    }
    for (int l = 1; l < L; ++l) {
        if (l == L - 1 && clamp_top) break;   // a clamped top is never updated (Layer.cs:275)
        if (upd.empty() || upd.back().n == kMaxProblems) { upd.emplace_back(); upd.back().n = 0; }
        ProblemSet& ps = upd.back();
        Problem& p = ps.p[ps.n++];
        std::memset(&p, 0, sizeof p);
        p.A = w->D[l];
        p.lda = m->P[l - 1];
        p.B = tile.wd ? m->WTpk[l] : m->WT[l];
        p.ldb = m->P[l - 1];
        p.M = batch;
        p.N = m->s[l];
        p.K = m->P[l - 1];
        p.tiles_m = tm;
        p.tiles_n = (p.N + tile.n - 1) / tile.n;
        p.tiles = p.tiles_m * p.tiles_n;
        p.ldo = m->P[l];
        p.m = w->M[l];
        p.mop = m->dtype == PCD_F32 ? nullptr : w->S[l];
        p.eself = l <= L - 2 ? w->E[l] : nullptr;
    }
    SplitScratch sc;
    sc.part = w->split_part;
    sc.count = w->split_count;
    sc.budget = split_part_tiles(m);
    const int smin = m->split_min > 0 ? m->split_min : tile.m == 32 ? kSplitMinStagesKsw : kSplitMinStages;
    assign_split(m->cus, m->split_k, m->dtype, tile, sc, err, smin);
    assign_split(m->cus, m->split_k, m->dtype, tile, sc, upd, smin);
    *nslots = slot;
}

int auto_k_stagger(int nk, bool one_row_tile) {
    return std::max(2, std::min(kMaxKStagger, nk / (one_row_tile ? 2 : 4)));
}

PhaseArgs base_args(const pcd_model* m, const Workspace* w, int batch, int nslots) {
    PhaseArgs a;
    std::memset(&a, 0, sizeof a);
    a.act = m->act;
    a.eta = m->eta;
    a.act_reg = m->act_reg;
    a.alpha = 1.f;
    a.energy_part = w->energy_part;
    a.ldp = w->cap;
    a.nslots = nslots;
    a.batch = batch;
    a.tile_order = m->tile_order;
    a.k_stagger = m->k_stagger;
    return a;
}

// One settling to enqueue: rows, steps, tile and the per-call variants.
struct RelaxSpec {
    int batch = 0, steps = 0;
    Tile tile{0, 0};
    int clamp_top = 0;              // layer L-1 holds rows staged by the caller and is never updated
    int keep_hidden = 0;            // layers 1..L-2 start from rows staged by the caller, not from zero
    int persistent = 0;             // the step loop as one persistent launch (see persistent_fits)
    float* energy_out = nullptr;    // [steps x batch] per-row energies (nullable)
    // ragged early exit (row_req null: fixed steps for every row)
    const int* row_req = nullptr;
    int* done_at = nullptr;
    const int* row_offsets = nullptr;
    int requests = 0, exit_rule = 0;
    float exit_thr = 0.f;
    float* prev_energy = nullptr;
    float* last_energy = nullptr;
};

// With a timer, each phase launch is bracketed by HIP events (eager only).
struct PhaseTimer {
    std::vector<std::pair<hipEvent_t, hipEvent_t>> err, upd;
};

// Waits for the timed launches, stores the average error- and update-phase
// durations in the model, and destroys the events (also after a failure).
int collect_timer(pcd_model* m, PhaseTimer& timer, hipStream_t s) {
    hipError_t e = hipStreamSynchronize(s);
    double te = 0, tu = 0;
    for (size_t i = 0; i < timer.upd.size() && e == hipSuccess; ++i) {
        float a = 0, b = 0;
        e = hipEventElapsedTime(&a, timer.err[i].first, timer.err[i].second);
        if (e == hipSuccess) e = hipEventElapsedTime(&b, timer.upd[i].first, timer.upd[i].second);
        te += a;
        tu += b;
    }
    for (auto& p : timer.err) {
        (void)hipEventDestroy(p.first);
        (void)hipEventDestroy(p.second);
    }
    for (auto& p : timer.upd) (void)hipEventDestroy(p.second);  // its first event is the error phase's second
    if (e != hipSuccess) return from_hip(e, "phase timing");
    m->prof_launches = (int)timer.upd.size();
    m->prof_err_ms = m->prof_launches ? (float)(te / m->prof_launches) : 0.f;
    m->prof_upd_ms = m->prof_launches ? (float)(tu / m->prof_launches) : 0.f;
    return PCD_SUCCESS;
}

// The phases' common arguments for a settling (t and energy_out are set per
// launch).
PhaseArgs relax_args(const pcd_model* m, const Workspace* w, const RelaxSpec& r, int nslots) {
    PhaseArgs args = base_args(m, w, r.batch, nslots);
    if (args.k_stagger == kKStaggerAuto) {
        // the settling phases' longest K sweep at this tile (padded sizes are
        // both phases' K)
        const int maxp = *std::max_element(m->P.begin(), m->P.end());
        args.k_stagger = auto_k_stagger(maxp / stage_k(m->dtype, r.tile), r.batch <= r.tile.m);
    }
    args.row_req = r.row_req;
    args.done_at = r.done_at;
    // Non-temporal epilogue stores and fp32 state loads for 16-bit models
    // (same box, two runs each; stores: c5 +2.1%, c5s +5.4%, c3 +0.3%; loads on
    // top: c5 +1.4%, c3 +0.35%, c5s unchanged).  fp32 models keep ordinary
    // ones (c2 -1.4% with the stores, -1% with the loads: its 4 MB states are
    // read again from the caches by the next phase; c1 and c4 unchanged).
    args.nt_store = m->nt_store >= 0 ? m->nt_store : m->dtype != PCD_F32;
    args.nt_load = m->nt_load >= 0 ? m->nt_load : m->dtype != PCD_F32;
    const bool need_energy = r.energy_out != nullptr || r.row_req != nullptr;
    if (!need_energy) args.energy_part = nullptr;
    return args;
}

// Zero the free states, FFG warm start (Network.cs:121-131), then the step
// loop.  Layer 0 (and, with clamp_top, layer L-1) must already hold its rows.
int enqueue_relax(pcd_model* m, Workspace* w, const RelaxSpec& r, hipStream_t s, PhaseTimer* timer) {
    const int L = m->L;
    const int batch = r.batch;
    const Tile tile = r.tile;
    int st;
    ZeroBatch zb;
    for (int l = 1; l < L; ++l) {
        if (l == L - 1 && r.clamp_top) break;
        if (l <= L - 2 && r.keep_hidden) continue;
        if ((st = zb.add(w->M[l], (size_t)w->cap * m->P[l] * 4, s))) return st;
        if (w->S[l] && (st = zb.add(w->S[l], (size_t)w->cap * m->P[l] * op_bytes(m->dtype), s))) return st;
    }
    if ((st = zb.flush(s))) return st;
    std::vector<ProblemSet> err, upd;
    int nslots = 0;
    build_phase_sets(m, w, batch, tile, r.clamp_top, err, upd, &nslots);
    const PhaseArgs args = relax_args(m, w, r, nslots);

    if (m->ffg) {
        for (int l = L - 1; l >= 2; --l) {
            ProblemSet ps;
            std::memset(&ps, 0, sizeof ps);
            ps.n = 1;
            Problem& p = ps.p[0];
            p.A = state_operand(m, w, l);
            p.lda = m->P[l];
            p.B = tile.wd ? m->Wpk[l] : m->W[l];
            p.ldb = m->P[l];
            p.M = batch;
            p.N = m->s[l - 1];
            p.K = m->P[l];
            p.tiles_m = (batch + tile.m - 1) / tile.m;
            p.tiles_n = (p.N + tile.n - 1) / tile.n;
            p.tiles = p.tiles_m * p.tiles_n;
            p.ldo = m->P[l - 1];
            p.bias = m->bias[l];
            p.m = w->M[l - 1];
            p.dout = m->dtype == PCD_F32 ? nullptr : w->S[l - 1];
            PhaseArgs fa = args;
            fa.row_req = nullptr;
            if ((st = launch_phase(m->dtype, tile, EPI_FFG, ps, fa, s))) return st;
        }
    }
    // Ragged: before each step, list the row tiles that still hold a running
    // row; both phases of the step then deal only those over the XCDs.
    const bool tile_list = r.row_req != nullptr && m->ragged_tiles && (batch + tile.m - 1) / tile.m <= kMaxActTiles;
    for (int t = 0; t < r.steps; ++t) {
        PhaseArgs a = args;
        a.t = t;
        a.energy_out = nullptr;
        if (tile_list) {
            hipLaunchKernelGGL(active_tiles_kernel, dim3(1), dim3(kActTilesThreads), 0, s, r.row_offsets,
                               (const int*)r.done_at, r.requests, batch, tile.m, t, w->act_tm, w->act_count);
            if ((st = from_hip(hipGetLastError(), "active_tiles_kernel launch"))) return st;
            a.act_tm = w->act_tm;
            a.act_count = w->act_count;
        }
        hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr;
        if (timer) {
            HIP_TRY(hipEventCreate(&e0));
            HIP_TRY(hipEventCreate(&e1));
            HIP_TRY(hipEventCreate(&e2));
            HIP_TRY(hipEventRecord(e0, s));
        }
        for (auto& ps : err)
            if ((st = launch_phase(m->dtype, tile, EPI_ERROR, ps, a, s))) return st;
        if (timer) HIP_TRY(hipEventRecord(e1, s));
        if (r.row_req && r.requests == batch) {
            // every request is one row (offsets increase strictly): a thread per request
            const int grid = std::min((batch + 255) / 256, 1024);
            hipLaunchKernelGGL(exit_rows_kernel, dim3(grid), dim3(256), 0, s, (const float*)w->energy_part, w->cap,
                               nslots, r.requests, r.done_at, r.prev_energy, r.last_energy, t, r.exit_rule,
                               r.exit_thr);
            if ((st = from_hip(hipGetLastError(), "exit_rows_kernel launch"))) return st;
        } else if (r.row_req) {
            hipLaunchKernelGGL(exit_kernel, dim3(r.requests), dim3(256), 0, s, (const float*)w->energy_part, w->cap,
                               nslots, r.row_offsets, r.done_at, r.prev_energy, r.last_energy, t, r.exit_rule,
                               r.exit_thr);
            if ((st = from_hip(hipGetLastError(), "exit_kernel launch"))) return st;
        }
        a.energy_out = r.energy_out;
        if (upd.empty() && r.energy_out) {
            // No free layer to update: reduce the step's row energies on their own.
            const int grid = std::min((batch + 255) / 256, 1024);
            hipLaunchKernelGGL(energy_rows_kernel, dim3(grid), dim3(256), 0, s, (const float*)w->energy_part,
                               w->cap, nslots, r.energy_out + (size_t)t * batch, batch);
            if ((st = from_hip(hipGetLastError(), "energy_rows_kernel launch"))) return st;
        }
        bool first = true;
        for (auto& ps : upd) {
            PhaseArgs ua = a;
            if (!first) ua.energy_out = nullptr;
            first = false;
            if ((st = launch_phase(m->dtype, tile, EPI_UPDATE, ps, ua, s))) return st;
        }
        if (timer) {
            HIP_TRY(hipEventRecord(e2, s));
            timer->err.push_back({e0, e1});
            timer->upd.push_back({e1, e2});
        }
    }
    return PCD_SUCCESS;
}

// The cached graph of the T-step loop described by r (its energy buffer is the
// plan's own when want_energy is set), captured on first use.
Plan* get_plan(pcd_model* m, Workspace* w, const RelaxSpec& r, int want_energy, int* status) {
    *status = PCD_SUCCESS;
    const int requests = r.row_req ? r.requests : 0;
    for (auto& p : w->plans)
        if (p->batch == r.batch && p->steps == r.steps && p->want_energy == want_energy &&
            p->clamp_top == r.clamp_top && p->keep_hidden == r.keep_hidden && same_tile(p->tile, r.tile) &&
            p->requests == requests && (requests == 0 || (p->exit_rule == r.exit_rule &&
                                                          std::memcmp(&p->exit_thr, &r.exit_thr, 4) == 0))) {
            p->last_use = ++m->clock;
            return p.get();
        }
    if (w->plans.size() >= 8) {  // evict the least recently used plan
        auto it = std::min_element(w->plans.begin(), w->plans.end(),
                                   [](const auto& a, const auto& b) { return a->last_use < b->last_use; });
        // Its last launch may still be queued on the workspace's stream (the
        // relax calls return without waiting): let it finish before the
        // executable graph and its energy buffer go.
        hipError_t e = hipStreamSynchronize(w->stream);
        if (e != hipSuccess) { *status = from_hip(e, "hipStreamSynchronize (plan eviction)"); return nullptr; }
        w->plans.erase(it);
    }
    std::unique_ptr<Plan> p(new Plan());
    p->batch = r.batch;
    p->steps = r.steps;
    p->want_energy = want_energy;
    p->clamp_top = r.clamp_top;
    p->keep_hidden = r.keep_hidden;
    p->tile = r.tile;
    p->requests = requests;
    p->exit_rule = requests ? r.exit_rule : 0;
    p->exit_thr = requests ? r.exit_thr : 0.f;
    p->last_use = ++m->clock;
    if (want_energy) {   // on any failure below, ~Plan releases what was made
        hipError_t e = hipMalloc(&p->energy_out, (size_t)r.steps * r.batch * 4);
        if (e != hipSuccess) { *status = from_hip(e, "hipMalloc(energy)"); return nullptr; }
    }
    hipStream_t cs = w->capture;
    std::unique_lock<std::mutex> no_legacy(legacy_stream_mu());   // no legacy-stream call while recording
    hipError_t e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) { *status = from_hip(e, "hipStreamBeginCapture"); return nullptr; }
    RelaxSpec rc = r;
    if (want_energy) rc.energy_out = p->energy_out;
    int st = enqueue_relax(m, w, rc, cs, nullptr);
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(cs, &g);
    no_legacy.unlock();
    if (st) { if (g) (void)hipGraphDestroy(g); *status = st; return nullptr; }
    if (e != hipSuccess) { *status = from_hip(e, "hipStreamEndCapture"); return nullptr; }
    p->graph = g;
    e = hipGraphInstantiate(&p->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { *status = from_hip(e, "hipGraphInstantiate"); return nullptr; }
    w->plans.push_back(std::move(p));
    return w->plans.back().get();
}

// A fixed-step fp32 settling whose phases deal at most two workgroups per CU
// (its launches, not its tiles, bound it) runs as one persistent launch:
// option `persistent` on, no profiling, 64 x 64 tiles, and each phase's
// problems fit the kernel argument.
bool persistent_fits(const pcd_model* m, Tile tile, const std::vector<ProblemSet>& err,
                     const std::vector<ProblemSet>& upd) {
    if (!m->persistent || m->profile || m->dtype != PCD_F32 || tile.m != 64 || tile.n != 64) return false;
    if (err.size() != 1 || upd.size() != 1) return false;
    if (err[0].n > kMaxPersistProblems || upd[0].n > kMaxPersistProblems) return false;
    const int lim = 2 * m->cus;
    return phase_grid(err[0], m->tile_order) <= lim && phase_grid(upd[0], m->tile_order) <= lim;
}

// The settling r (fixed steps, no ragged rows) as one persistent launch, when
// persistent_fits allows it; returns false (nothing enqueued) otherwise.  The
// states are zeroed and the FFG sweep runs as in enqueue_relax, then
// persistent_relax_kernel runs the step loop with grid barriers between the
// phases.  The call waits for the settling and reads the barrier's give-up
// flag: *status is PCD_HIP_ERROR if a barrier gave up.
bool run_persistent(pcd_model* m, Workspace* w, const RelaxSpec& r, hipStream_t s, int* status) {
    std::vector<ProblemSet> err, upd;
    int nslots = 0;
    build_phase_sets(m, w, r.batch, r.tile, r.clamp_top, err, upd, &nslots);
    if (!persistent_fits(m, r.tile, err, upd)) return false;
    // A caller capturing its stream into a graph gets the per-phase launches
    // (this form waits for the settling, which a capture cannot).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
    // workgroups of the launch: a multiple of the XCD count, all resident at once
    const int cap = persistent_blocks_per_cu() * m->cus / kXcds * kXcds;
    const int err_grid = phase_grid(err[0], m->tile_order), upd_grid = phase_grid(upd[0], m->tile_order);
    int nw = m->persist_grid > 0 ? m->persist_grid : (std::max(err_grid, upd_grid) + kXcds - 1) / kXcds * kXcds;
    if (nw > cap) nw = cap;
    if (nw < kXcds) return false;   // the kernel cannot be resident (no occupancy)
    // zero the free states and run the FFG sweep
    RelaxSpec r0 = r;
    r0.steps = 0;
    if ((*status = enqueue_relax(m, w, r0, s, nullptr))) return true;
    PersistArgs pa;
    std::memset(&pa, 0, sizeof pa);
    for (int i = 0; i < err[0].n; ++i) pa.err_p[i] = err[0].p[i];
    for (int i = 0; i < upd[0].n; ++i) pa.upd_p[i] = upd[0].p[i];
    pa.err = relax_args(m, w, r, nslots);
    pa.upd = pa.err;
    pa.err.energy_out = nullptr;
    pa.upd.energy_out = r.energy_out;
    pa.err_n = err[0].n;
    pa.upd_n = upd[0].n;
    pa.err_grid = err_grid;
    pa.upd_grid = upd_grid;
    pa.steps = r.steps;
    int* sync = (int*)w->persist;
    pa.sync.count = sync;
    pa.sync.error = sync + 1;
    pa.sync.spin_limit = m->persist_spin;
    if ((*status = launch_zero(sync, kPersistBytes, s))) return true;
    if ((*status = from_hip(launch_persistent_tile<float, 64, 64>(pa, nw, s), "persistent_relax_kernel launch")))
        return true;
    int flag = 0;
    hipError_t e = hipMemcpyAsync(&flag, sync + 1, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if ((*status = from_hip(e, "persistent settling")) != PCD_SUCCESS) return true;
    if (flag) {
        // Workgroups that left at a barrier skipped their units, while others
        // that saw every arrival went on: a split tile may have some of its
        // ranges counted and never reach the range that resets its counter.
        // The counters must read zero for the next launch of any kind.
        int zst = launch_zero(w->split_count, split_count_bytes(m), s);
        if (!zst) zst = from_hip(hipStreamSynchronize(s), "split counter reset");
        *status = zst ? zst
                      : fail(PCD_HIP_ERROR, "persistent settling: a barrier gave up after %d polls (%d workgroups)",
                             m->persist_spin, nw);
    }
    return true;
}

// A fixed-step settling of `batch` staged rows (layer 0, and the top with
// clamp_top): eager with per-phase timing under the profile option, else the
// cached graph of the T-step loop.  *energy receives the buffer holding the
// [steps x batch] row energies when want_energy is set (the caller's
// `caller_energy` or the plan's own), valid once the stream reaches it.
int run_relax(pcd_model* m, Workspace* w, int batch, int steps, int clamp_top, int want_energy, float* caller_energy,
              hipStream_t s, const float** energy, int keep_hidden = 0) {
    RelaxSpec r;
    r.batch = batch;
    r.steps = steps;
    r.tile = choose_tile(m, batch);
    r.clamp_top = clamp_top;
    r.keep_hidden = keep_hidden;
    *energy = nullptr;
    if (!want_energy || caller_energy) {
        r.energy_out = want_energy ? caller_energy : nullptr;
        int st = PCD_SUCCESS;
        if (run_persistent(m, w, r, s, &st)) {
            if (!st) *energy = r.energy_out;
            return st;
        }
        r.energy_out = nullptr;
    }
    if (m->profile || !m->use_graph) {
        float* buf = caller_energy;
        if (want_energy && !buf) return fail(PCD_INVALID_VALUE, "run_relax: energy buffer missing");
        r.energy_out = want_energy ? buf : nullptr;
        PhaseTimer timer;
        int st = enqueue_relax(m, w, r, s, m->profile ? &timer : nullptr);
        if (m->profile) {
            int st2 = collect_timer(m, timer, s);
            if (!st) st = st2;
        }
        if (st) return st;
        *energy = r.energy_out;
        return PCD_SUCCESS;
    }
    int st = PCD_SUCCESS;
    Plan* p = get_plan(m, w, r, want_energy, &st);
    if (!p) return st;
    HIP_TRY(hipGraphLaunch(p->exec, s));
    *energy = p->energy_out;
    return PCD_SUCCESS;
}

// Drops every cached graph of the model, once the streams that may still be
// running one of them have drained.
int drop_plans(pcd_model* m) {
    for (auto& w : m->ws) {
        if (w->plans.empty()) continue;
        HIP_TRY(hipStreamSynchronize(w->stream));
        w->plans.clear();
    }
    return PCD_SUCCESS;
}

int check_model(pcd_model* m) {
    if (!m) return fail(PCD_NOT_INITIALIZED, "null model");
    return PCD_SUCCESS;
}

}  // namespace

// ======================================================================= ABI

extern "C" {

int pcd_version(int* version) {
    if (!version) return fail(PCD_INVALID_VALUE, "null pointer");
    *version = 100;  // 0.1.0
    return PCD_SUCCESS;
}

int pcd_last_error(char* buf, size_t len) {
    if (!buf || len == 0) return fail(PCD_INVALID_VALUE, "pcd_last_error: empty buffer");
    std::snprintf(buf, len, "%s", g_last_error.c_str());
    return PCD_SUCCESS;
}

int pcd_get_device_count(int* count) {
    if (!count) return fail(PCD_INVALID_VALUE, "pcd_get_device_count: null pointer");
    *count = 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(PCD_NO_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
    }
    *count = n;
    return n > 0 ? PCD_SUCCESS : fail(PCD_NO_DEVICE, "no HIP device");
}

int pcd_set_device(int device) {
    HIP_TRY(hipSetDevice(device));
    return PCD_SUCCESS;
}

int pcd_get_device(int* device) {
    if (!device) return fail(PCD_INVALID_VALUE, "null pointer");
    HIP_TRY(hipGetDevice(device));
    return PCD_SUCCESS;
}

int pcd_device_synchronize(void) {
    HIP_TRY(device_sync());
    return PCD_SUCCESS;
}

// ----------------------------------------------------------------- memory

int pcd_malloc_async(void** ptr, size_t bytes, void* stream) { return pool_alloc(ptr, bytes, (hipStream_t)stream); }

int pcd_free_async(void* ptr, void* stream) { return pool_free(ptr, (hipStream_t)stream); }

int pcd_host_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(PCD_INVALID_VALUE, "pcd_host_alloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return PCD_SUCCESS;
    int b = bucket_of(bytes);
    Pool& P = pool();
    {
        std::lock_guard<std::mutex> g(P.mu);
        auto& v = P.host_free[b];
        if (!v.empty()) {
            *ptr = v.back();
            v.pop_back();
            P.host_live[*ptr] = b;
            return PCD_SUCCESS;
        }
    }
    void* p = nullptr;
    HIP_TRY(hipHostMalloc(&p, (size_t)1 << b, hipHostMallocDefault));
    std::lock_guard<std::mutex> g(P.mu);
    P.host_live[p] = b;
    *ptr = p;
    return PCD_SUCCESS;
}

int pcd_host_free(void* ptr) {
    if (!ptr) return PCD_SUCCESS;
    Pool& P = pool();
    std::lock_guard<std::mutex> g(P.mu);
    auto it = P.host_live.find(ptr);
    if (it == P.host_live.end()) return fail(PCD_INVALID_VALUE, "pcd_host_free: pointer not from pcd_host_alloc");
    int b = it->second;
    P.host_live.erase(it);
    auto& v = P.host_free[b];
    if (v.size() < Pool::kMaxCached) {
        v.push_back(ptr);
        return PCD_SUCCESS;
    }
    HIP_TRY(hipHostFree(ptr));
    return PCD_SUCCESS;
}

int pcd_trim_pools(void) {
    HIP_TRY(device_sync());
    Pool& P = pool();
    std::lock_guard<std::mutex> g(P.mu);
    for (auto& kv : P.free_blocks)
        for (void* p : kv.second) {
            (void)hipFree(p);
            P.synchronous.erase(p);
        }
    P.free_blocks.clear();
    for (auto& kv : P.host_free)
        for (void* p : kv.second) (void)hipHostFree(p);
    P.host_free.clear();
    return PCD_SUCCESS;
}

static int to_kind(int kind, hipMemcpyKind* out) {
    switch (kind) {
    case PCD_HOST_TO_HOST: *out = hipMemcpyHostToHost; return PCD_SUCCESS;
    case PCD_HOST_TO_DEVICE: *out = hipMemcpyHostToDevice; return PCD_SUCCESS;
    case PCD_DEVICE_TO_HOST: *out = hipMemcpyDeviceToHost; return PCD_SUCCESS;
    case PCD_DEVICE_TO_DEVICE: *out = hipMemcpyDeviceToDevice; return PCD_SUCCESS;
    case PCD_MEMCPY_DEFAULT: *out = hipMemcpyDefault; return PCD_SUCCESS;
    default: return fail(PCD_INVALID_VALUE, "bad memcpy kind %d", kind);
    }
}

int pcd_memcpy(void* dst, const void* src, size_t bytes, int kind) {
    hipMemcpyKind k;
    if (int st = to_kind(kind, &k)) return st;
    if (bytes == 0) return PCD_SUCCESS;
    if (!dst || !src) return fail(PCD_INVALID_VALUE, "pcd_memcpy: null pointer");
    HIP_TRY(sync_memcpy(dst, src, bytes, k));
    return PCD_SUCCESS;
}

int pcd_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
    hipMemcpyKind k;
    if (int st = to_kind(kind, &k)) return st;
    if (bytes == 0) return PCD_SUCCESS;
    if (!dst || !src) return fail(PCD_INVALID_VALUE, "pcd_memcpy_async: null pointer");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, (hipStream_t)stream));
    return PCD_SUCCESS;
}

int pcd_memset_async(void* dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return PCD_SUCCESS;
    if (!dst) return fail(PCD_INVALID_VALUE, "pcd_memset_async: null pointer");
    HIP_TRY(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return PCD_SUCCESS;
}

// ---------------------------------------------------------- streams, events

int pcd_stream_create(void** stream) {
    if (!stream) return fail(PCD_INVALID_VALUE, "null pointer");
    hipStream_t s = nullptr;
    HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return PCD_SUCCESS;
}

int pcd_stream_destroy(void* stream) {
    if (!stream) return PCD_SUCCESS;
    HIP_TRY(hipStreamDestroy((hipStream_t)stream));
    return PCD_SUCCESS;
}

int pcd_stream_synchronize(void* stream) {
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return PCD_SUCCESS;
}

int pcd_event_create(void** event) {
    if (!event) return fail(PCD_INVALID_VALUE, "null pointer");
    hipEvent_t e = nullptr;
    HIP_TRY(hipEventCreate(&e));
    *event = e;
    return PCD_SUCCESS;
}

int pcd_event_record(void* event, void* stream) {
    if (!event) return fail(PCD_INVALID_VALUE, "null event");
    HIP_TRY(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return PCD_SUCCESS;
}

int pcd_event_synchronize(void* event) {
    if (!event) return PCD_SUCCESS;
    HIP_TRY(hipEventSynchronize((hipEvent_t)event));
    return PCD_SUCCESS;
}

int pcd_event_destroy(void* event) {
    if (!event) return PCD_SUCCESS;
    HIP_TRY(hipEventDestroy((hipEvent_t)event));
    return PCD_SUCCESS;
}

int pcd_event_elapsed_ms(float* ms, void* start, void* end) {
    if (!ms || !start || !end) return fail(PCD_INVALID_VALUE, "null pointer");
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return PCD_SUCCESS;
}

// -------------------------------------------------------------------- GEMM

// Output tile of a provider GEMM: 256 x 256 (16-bit operands) while it still
// gives every CU a tile, then 128 x 128 while that does, else 64 x 64 (whose
// few tiles split-K then spreads over the CUs); fp32 products with fewer
// 64 x 64 tiles than CUs take the K-shared 32 x 32 tile.  `batch` products of
// the same shape count together, but only among the tiles that fit one
// product: a tile wider than the product (rounded up to 64) in either
// dimension would be mostly padding, in MFMA work and in packed operand
// memory, however many products there are.
// Provider outputs of at least this many bytes (twice the chip's L2) are
// stored non-temporally: a caller reads them long after the L2 has turned over.
constexpr size_t kGemmNtBytes = (size_t)64 << 20;

static Tile choose_gemm_tile(int dtype, int m, int n, int cus, int batch = 1) {
    auto tiles = [&](int t) { return (long)batch * ((m + t - 1) / t) * ((n + t - 1) / t); };
    auto fits = [&](int t) { return t <= (int)round_up(m, 64) && t <= (int)round_up(n, 64); };
    if (dtype != PCD_F32 && fits(256) && tiles(256) >= cus) return Tile{256, 256};
    if (fits(128) && tiles(128) >= cus) return Tile{128, 128};
    if (dtype == PCD_F32 && tiles(64) < cus) return Tile{32, 32};
    return Tile{64, 64};
}

static int gemm_common(int dtype, const void* dA, const void* dB, float* dC, int m, int k, int n, int trans_a,
                       int trans_b, float beta, void* stream_) {
    if (!dA || !dB || !dC) return fail(PCD_INVALID_VALUE, "pcd_gemm: null pointer");
    if (m < 1 || k < 1 || n < 1) return fail(PCD_INVALID_VALUE, "pcd_gemm: bad shape %d x %d x %d", m, k, n);
    hipStream_t s = (hipStream_t)stream_;
    int dev = 0, cus = 256;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const Tile tile = choose_gemm_tile(dtype, m, n, cus);
    const int mp = (int)round_up(m, tile.m), np = (int)round_up(n, tile.n), kp = (int)round_up(k, kFeatPad);
    const int ob = op_bytes(dtype);
    // An operand already K-contiguous, with whole tiles of rows, K a whole
    // number of stages and 16-byte aligned rows, is read where it lies; any
    // other is packed into zero-padded scratch.
    auto aligned = [&](const void* p) { return ((uintptr_t)p % 16) == 0; };
    const bool direct_a = !trans_a && m == mp && k == kp && aligned(dA);
    const bool direct_b = trans_b && n == np && k == kp && aligned(dB);
    // B in Gemm.MatMul's own row-major [k x n] layout, with whole tiles of
    // columns and K a whole number of stages, is read where it lies too, on the
    // 16-bit tiles that transpose it in LDS (EPI_PLAIN_KN).
    // So is a transposed A (physical [k x m]) on those tiles (EPI_PLAIN_MK).
    // Except that the transposing reads cost the 128 x 128 tile about a fifth
    // of its time, more than packing an operand a quarter the other's size or
    // smaller takes (512 x 8192 x 8192 bf16, A transposed: 0.089 ms in place,
    // 0.081 packed; the other tiles lose 2-5% and read in place).
    const bool small_a = tile.m == 128 && (size_t)m * 4 <= (size_t)n;
    const bool small_b = tile.m == 128 && (size_t)n * 4 <= (size_t)m;
    const bool kn_b = !trans_b && !small_b && kn_tile(ob, tile.m, tile.n, false) && n == np && k == kp && aligned(dB);
    const bool mk_a = trans_a && !small_a && kn_tile(ob, tile.m, tile.n, false) && m == mp && k == kp && aligned(dA);
    void *pa = nullptr, *pb = nullptr;
    int st = PCD_SUCCESS;
    auto release = [&]() {
        if (pa && !direct_a && !mk_a) pool_free(pa, s);
        if (pb && !direct_b && !kn_b) pool_free(pb, s);
    };
    const int src_f32 = dtype == PCD_F32;
    auto pack = [&](const void* src, int rows, int cols, int trans, void* dst, int prow, int pcol) -> int {
        switch (dtype) {
        case PCD_F32: pack_op<float>(s, src, src_f32, rows, cols, trans, dst, prow, pcol, pcol); break;
        case PCD_BF16: pack_op<bf16_t>(s, src, src_f32, rows, cols, trans, dst, prow, pcol, pcol); break;
        default: pack_op<f16_t>(s, src, src_f32, rows, cols, trans, dst, prow, pcol, pcol); break;
        }
        return from_hip(hipGetLastError(), "pack_kernel launch");
    };
    // op(A) [m x k]: physical [m x k], or [k x m] when transposed.
    // The kernel's B operand is op(B)^T [n x k]: physical B is [k x n] (read
    // transposed) or, with trans_b, already [n x k].
    if (direct_a || mk_a) pa = (void*)dA;
    else if (!(st = pool_alloc(&pa, (size_t)mp * kp * ob, s))) st = pack(dA, m, k, trans_a, pa, mp, kp);
    if (!st) {
        if (direct_b || kn_b) pb = (void*)dB;
        else if (!(st = pool_alloc(&pb, (size_t)np * kp * ob, s))) st = pack(dB, n, k, trans_b ? 0 : 1, pb, np, kp);
    }
    std::vector<ProblemSet> sets(1);
    std::memset(&sets[0], 0, sizeof(ProblemSet));
    sets[0].n = 1;
    Problem& p = sets[0].p[0];
    p.A = pa;
    p.lda = mk_a ? m : kp;   // the row pitch of a transposed A, else of the K-contiguous rows
    p.B = pb;
    p.ldb = kn_b ? n : kp;   // the row pitch of row-major B, else of the K-contiguous copy
    p.M = m;
    p.N = n;
    p.K = kp;
    p.tiles_m = mp / tile.m;
    p.tiles_n = np / tile.n;
    p.tiles = p.tiles_m * p.tiles_n;
    p.ldo = n;
    p.m = dC;
    // Split-K scratch from the pool; the counters start at zero (a fill
    // kernel, so a captured call stays free of memset nodes).
    SplitScratch sc;
    void* part = nullptr;
    if (!st && tile.m * tile.n <= 128 * 128 && p.tiles * 2 <= cus) {
        sc.budget = cus;
        const size_t part_bytes = (size_t)sc.budget * 128 * 128 * 4, cnt_bytes = split_count_bytes((int)sc.budget);
        if (!(st = pool_alloc(&part, part_bytes + cnt_bytes, s))) {
            sc.part = (float*)part;
            sc.count = (int*)((char*)part + part_bytes);
            st = launch_zero(sc.count, cnt_bytes, s);
        }
    }
    if (!st) assign_split(cus, 1, dtype, tile, sc, sets, tile.m == 32 ? kSplitMinStagesKsw : kSplitMinStages);
    PhaseArgs a;
    std::memset(&a, 0, sizeof a);
    a.alpha = 1.f;
    a.beta = beta;
    a.k_stagger = dtype == PCD_F32 ? 0 : auto_k_stagger(kp / stage_k(dtype, tile));
    a.nt_store = (size_t)m * n * 4 >= kGemmNtBytes;
    const int epi = mk_a ? (kn_b ? EPI_PLAIN_MKKN : EPI_PLAIN_MK) : (kn_b ? EPI_PLAIN_KN : EPI_PLAIN);
    if (!st) st = launch_phase(dtype, tile, epi, sets[0], a, s);
    release();
    if (part) {
        int st2 = pool_free(part, s);
        if (!st) st = st2;
    }
    return st;
}

// Strided batched GEMM: C_i = A_i B_i for i < batch, row-major, A_i [m x k] at
// dA + i m k, B_i [k x n] at dB + i k n, C_i [m x n] at dC + i m n.  Both
// operands of every item are packed K-contiguous in one launch each; the
// items are the problems of grouped phase launches (kMaxProblems per launch),
// their tiles dealt over the XCDs together.
static int gemm_batched_common(int dtype, const void* dA, const void* dB, float* dC, int batch, int m, int k, int n,
                               void* stream_) {
    if (!dA || !dB || !dC) return fail(PCD_INVALID_VALUE, "pcd_gemm_batched: null pointer");
    if (batch < 1 || m < 1 || k < 1 || n < 1)
        return fail(PCD_INVALID_VALUE, "pcd_gemm_batched: bad shape %d x (%d x %d x %d)", batch, m, k, n);
    hipStream_t s = (hipStream_t)stream_;
    int dev = 0, cus = 256;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const Tile tile = choose_gemm_tile(dtype, m, n, cus, batch);
    const int mp = (int)round_up(m, tile.m), np = (int)round_up(n, tile.n), kp = (int)round_up(k, kFeatPad);
    const int ob = op_bytes(dtype);
    const size_t a_item = (size_t)mp * kp * ob, b_item = (size_t)np * kp * ob;
    // Each B_i [k x n] is read where it lies (EPI_PLAIN_KN) when the tile has
    // that form, its columns fill whole tiles, K is a whole number of stages and
    // every item starts 16-byte aligned.
    // (and not on the 128 x 128 tile when B_i is a quarter of A_i or smaller: see gemm_common)
    const bool kn_b = kn_tile(ob, tile.m, tile.n, false) && n == np && k == kp && (uintptr_t)dB % 16 == 0 &&
                      !(tile.m == 128 && (size_t)n * 4 <= (size_t)m);
    void *pa = nullptr, *pb = nullptr;
    int st = pool_alloc(&pa, a_item * batch, s);
    if (!st && !kn_b) st = pool_alloc(&pb, b_item * batch, s);
    auto pack = [&](const void* src, int rows, int cols, int trans, void* dst, int prow, int pcol) -> int {
        const int grid = (int)std::min<size_t>(((size_t)batch * prow * pcol + 255) / 256, 16384);
        const int f32 = dtype == PCD_F32;
        switch (dtype) {
        case PCD_F32: hipLaunchKernelGGL(pack_batched_kernel<float>, dim3(grid), dim3(256), 0, s, src, f32, batch, rows, cols, trans, dst, prow, pcol); break;
        case PCD_BF16: hipLaunchKernelGGL(pack_batched_kernel<bf16_t>, dim3(grid), dim3(256), 0, s, src, f32, batch, rows, cols, trans, dst, prow, pcol); break;
        default: hipLaunchKernelGGL(pack_batched_kernel<f16_t>, dim3(grid), dim3(256), 0, s, src, f32, batch, rows, cols, trans, dst, prow, pcol); break;
        }
        return from_hip(hipGetLastError(), "pack_batched_kernel launch");
    };
    // the kernel's A is A_i [m x k]; its B is B_i^T [n x k] (B_i read transposed)
    if (!st) st = pack(dA, m, k, 0, pa, mp, kp);
    if (!st && !kn_b) st = pack(dB, n, k, 1, pb, np, kp);
    PhaseArgs a;
    std::memset(&a, 0, sizeof a);
    a.alpha = 1.f;
    a.beta = 0.f;
    a.k_stagger = dtype == PCD_F32 ? 0 : auto_k_stagger(kp / stage_k(dtype, tile));
    a.nt_store = (size_t)batch * m * n * 4 >= kGemmNtBytes;
    for (int i0 = 0; i0 < batch && !st; i0 += kMaxProblems) {
        ProblemSet ps;
        std::memset(&ps, 0, sizeof ps);
        ps.n = std::min(kMaxProblems, batch - i0);
        for (int q = 0; q < ps.n; ++q) {
            const size_t i = (size_t)(i0 + q);
            Problem& p = ps.p[q];
            p.A = (const char*)pa + i * a_item;
            p.lda = kp;
            p.B = kn_b ? (const void*)((const char*)dB + i * (size_t)k * n * ob) : (const void*)((const char*)pb + i * b_item);
            p.ldb = kn_b ? n : kp;
            p.M = m;
            p.N = n;
            p.K = kp;
            p.tiles_m = mp / tile.m;
            p.tiles_n = np / tile.n;
            p.tiles = p.tiles_m * p.tiles_n;
            p.ldo = n;
            p.m = dC + i * (size_t)m * n;
        }
        st = launch_phase(dtype, tile, kn_b ? EPI_PLAIN_KN : EPI_PLAIN, ps, a, s);
    }
    if (pa) {
        int st2 = pool_free(pa, s);
        if (!st) st = st2;
    }
    if (pb) {
        int st2 = pool_free(pb, s);
        if (!st) st = st2;
    }
    return st;
}

int pcd_gemm_f32_batched(const float* dA, const float* dB, float* dC, int batch, int m, int k, int n, void* stream) {
    return gemm_batched_common(PCD_F32, dA, dB, dC, batch, m, k, n, stream);
}

int pcd_gemm_bf16_batched(const uint16_t* dA, const uint16_t* dB, float* dC, int batch, int m, int k, int n,
                          void* stream) {
    return gemm_batched_common(PCD_BF16, dA, dB, dC, batch, m, k, n, stream);
}

int pcd_gemm_f16_batched(const uint16_t* dA, const uint16_t* dB, float* dC, int batch, int m, int k, int n,
                         void* stream) {
    return gemm_batched_common(PCD_F16, dA, dB, dC, batch, m, k, n, stream);
}

int pcd_gemm_f32(const float* dA, const float* dB, float* dC, int m, int k, int n, int trans_a, int trans_b,
                 float beta, void* stream) {
    return gemm_common(PCD_F32, dA, dB, dC, m, k, n, trans_a, trans_b, beta, stream);
}

int pcd_gemm_bf16(const uint16_t* dA, const uint16_t* dB, float* dC, int m, int k, int n, int trans_a, int trans_b,
                  float beta, void* stream) {
    return gemm_common(PCD_BF16, dA, dB, dC, m, k, n, trans_a, trans_b, beta, stream);
}

int pcd_gemm_f16(const uint16_t* dA, const uint16_t* dB, float* dC, int m, int k, int n, int trans_a, int trans_b,
                 float beta, void* stream) {
    return gemm_common(PCD_F16, dA, dB, dC, m, k, n, trans_a, trans_b, beta, stream);
}

// ---------------------------------------------------------------- PC model

int pcd_pc_model_create(const int* sizes, int levels, int activation, float eta, float act_reg, int ffg,
                        const float* const* W, const float* const* b, const float* precisions, int dtype,
                        pcd_model** out) {
    if (!out) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: null out pointer");
    *out = nullptr;
    if (!sizes || !precisions) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: null pointer");
    if (!W != !b) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: W and b must both be set or both be null");
    if (levels < 2) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: need at least 2 levels, got %d", levels);
    if (activation < PCD_ACT_LINEAR || activation > PCD_ACT_GELU)
        return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: unknown activation %d", activation);
    if (dtype != PCD_F32 && dtype != PCD_BF16 && dtype != PCD_F16)
        return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: unknown dtype %d", dtype);
    if (!(eta == eta) || !(act_reg >= 0.f)) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: bad eta/act_reg");
    for (int l = 0; l < levels; ++l) {
        if (sizes[l] < 1) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: sizes[%d] = %d", l, sizes[l]);
        if (!(precisions[l] > 0.f)) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: precision[%d] <= 0", l);
    }
    if (W)
        for (int l = 1; l < levels; ++l)
            if (!W[l - 1] || !b[l - 1]) return fail(PCD_INVALID_VALUE, "pcd_pc_model_create: null W/b for layer %d", l);
    int ndev = 0;
    if (int st = pcd_get_device_count(&ndev)) return st;

    std::unique_ptr<pcd_model> m(new pcd_model());
    HIP_TRY(hipGetDevice(&m->device));
    HIP_TRY(hipDeviceGetAttribute(&m->cus, hipDeviceAttributeMultiprocessorCount, m->device));
    m->L = levels;
    m->s.assign(sizes, sizes + levels);
    m->P.resize(levels);
    for (int l = 0; l < levels; ++l) m->P[l] = (int)round_up(sizes[l], kFeatPad);
    m->act = activation;
    m->ffg = ffg ? 1 : 0;
    m->dtype = dtype;
    m->k_stagger = dtype == PCD_F32 ? 0 : kKStaggerAuto;
    m->eta = eta;
    m->act_reg = act_reg;
    m->prec.assign(precisions, precisions + levels);
    m->W.assign(levels, nullptr);
    m->WT.assign(levels, nullptr);
    m->W32.assign(levels, nullptr);
    m->bias.assign(levels, nullptr);
    const int ob = op_bytes(dtype);
    std::vector<void*> owned;
    auto cleanup = [&]() { for (void* p : owned) (void)hipFree(p); };
    if (direct_eligible(m.get())) {
        m->Wpk.assign(levels, nullptr);
        m->WTpk.assign(levels, nullptr);
    }
    for (int l = 1; l < levels; ++l) {
        const int lo = sizes[l - 1], sz = sizes[l];
        const int Rlo = (int)round_up(lo, kRowPad), Rsz = (int)round_up(sz, kRowPad);
        int st;
        void *w = nullptr, *wt = nullptr, *bb = nullptr, *tmp = nullptr;
        if ((st = dev_alloc_zero(owned, &w, (size_t)Rlo * m->P[l] * ob)) ||
            (st = dev_alloc_zero(owned, &wt, (size_t)Rsz * m->P[l - 1] * ob)) ||
            (st = dev_alloc_zero(owned, &bb, (size_t)m->P[l - 1] * 4))) {
            cleanup();
            return st;
        }
        m->W[l] = w;
        m->WT[l] = wt;
        m->bias[l] = (float*)bb;
        if (!m->Wpk.empty()) {
            if ((st = dev_alloc_zero(owned, &m->Wpk[l], (size_t)Rlo * m->P[l] * ob)) ||
                (st = dev_alloc_zero(owned, &m->WTpk[l], (size_t)Rsz * m->P[l - 1] * ob))) {
                cleanup();
                return st;
            }
        }
        if (dtype != PCD_F32) {
            // fp32 masters, which the learning step updates (Network.LearnMixed's scheme)
            void* w32 = nullptr;
            if ((st = dev_alloc_zero(owned, &w32, (size_t)Rlo * m->P[l] * 4))) {
                cleanup();
                return st;
            }
            m->W32[l] = (float*)w32;
        }
        if (!W) continue;   // zero weights, to be filled by pcd_pc_model_load_record
        if ((st = dev_alloc_zero(owned, &tmp, (size_t)lo * sz * 4))) {
            cleanup();
            return st;
        }
        hipError_t e = sync_memcpy(tmp, W[l - 1], (size_t)lo * sz * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = sync_memcpy(bb, b[l - 1], (size_t)lo * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) { cleanup(); return from_hip(e, "sync_memcpy(weights)"); }
        // W_l as stored ([lo x sz] -> [Rlo x P_l]) and transposed ([sz x lo] -> [Rsz x P_{l-1}]).
        switch (dtype) {
        case PCD_F32:
            pack_op<float>(0, tmp, 1, lo, sz, 0, w, Rlo, m->P[l], m->P[l]);
            pack_op<float>(0, tmp, 1, sz, lo, 1, wt, Rsz, m->P[l - 1], m->P[l - 1]);
            break;
        case PCD_BF16:
            pack_op<bf16_t>(0, tmp, 1, lo, sz, 0, w, Rlo, m->P[l], m->P[l]);
            pack_op<bf16_t>(0, tmp, 1, sz, lo, 1, wt, Rsz, m->P[l - 1], m->P[l - 1]);
            break;
        default:
            pack_op<f16_t>(0, tmp, 1, lo, sz, 0, w, Rlo, m->P[l], m->P[l]);
            pack_op<f16_t>(0, tmp, 1, sz, lo, 1, wt, Rsz, m->P[l - 1], m->P[l - 1]);
            break;
        }
        if (m->W32[l])
            pack_op<float>(0, tmp, 1, lo, sz, 0, m->W32[l], Rlo,
                               m->P[l], m->P[l]);
        e = hipGetLastError();
        if (e == hipSuccess && (st = repack_direct(m.get(), l, 0))) { cleanup(); return st; }
        if (e == hipSuccess) e = device_sync();
        if (e != hipSuccess) { cleanup(); return from_hip(e, "weight packing"); }
        (void)hipFree(tmp);
        owned.pop_back();
    }
    *out = m.release();
    return PCD_SUCCESS;
}

int pcd_pc_model_destroy(pcd_model* m) {
    if (!m) return PCD_SUCCESS;
    (void)device_sync();
    for (auto& w : m->ws) free_workspace(*w);
    for (int l = 1; l < m->L; ++l) {
        (void)hipFree(m->W[l]);
        (void)hipFree(m->WT[l]);
        (void)hipFree(m->bias[l]);
        if (m->W32[l]) (void)hipFree(m->W32[l]);
        if (!m->Wpk.empty()) {
            (void)hipFree(m->Wpk[l]);
            (void)hipFree(m->WTpk[l]);
        }
    }
    delete m;
    return PCD_SUCCESS;
}

int pcd_pc_model_info(const pcd_model* m, int* levels, int* sizes, int max_sizes, int* dtype) {
    if (!m) return fail(PCD_NOT_INITIALIZED, "null model");
    if (levels) *levels = m->L;
    if (dtype) *dtype = m->dtype;
    if (sizes)
        for (int l = 0; l < m->L && l < max_sizes; ++l) sizes[l] = m->s[l];
    return PCD_SUCCESS;
}

int pcd_pc_set_option(pcd_model* m, const char* name, int value) {
    if (int st = check_model(m)) return st;
    if (!name) return fail(PCD_INVALID_VALUE, "null option name");
    std::lock_guard<std::mutex> g(m->mu);
    std::string n(name);
    if (n == "use_graph") m->use_graph = value ? 1 : 0;
    else if (n == "tile") {
        if (value != 0 && !tile_supported(Tile{value, value}))
            return fail(PCD_INVALID_VALUE, "tile must be 0, 32, 64, 128 or 256");
        m->tile_m = m->tile_n = value;
    } else if (n == "tile_n") {
        if (m->tile_m == 0 || !tile_supported(Tile{m->tile_m, value}))
            return fail(PCD_INVALID_VALUE, "tile_n: unsupported tile %d x %d (set tile first)", m->tile_m, value);
        m->tile_n = value;
    } else if (n == "profile") m->profile = value ? 1 : 0;
    else if (n == "split_k") m->split_k = value ? 1 : 0;
    else if (n == "tile_order") {
        if (value != TILE_INTERLEAVED && value != TILE_CONTIGUOUS)
            return fail(PCD_INVALID_VALUE, "tile_order must be 0 (interleaved) or 1 (contiguous)");
        m->tile_order = value;
    } else if (n == "ragged_tiles") m->ragged_tiles = value ? 1 : 0;
    else if (n == "persistent") m->persistent = value ? 1 : 0;
    else if (n == "split_min") {
        if (value < 0) return fail(PCD_INVALID_VALUE, "split_min must be >= 0 (0: automatic)");
        m->split_min = value;
    }
    else if (n == "persist_spin") {
        if (value < 1) return fail(PCD_INVALID_VALUE, "persist_spin must be >= 1");
        m->persist_spin = value;
    } else if (n == "persist_grid") {
        if (value < 0 || value % kXcds)
            return fail(PCD_INVALID_VALUE, "persist_grid must be 0 or a multiple of %d", kXcds);
        m->persist_grid = value;
    }
    else if (n == "ragged_order") m->ragged_order = value ? 1 : 0;
    else if (n == "nt_store" || n == "nt_load") {
        if (value < -1 || value > 1) return fail(PCD_INVALID_VALUE, "%s must be -1 (automatic), 0 or 1", name);
        (n == "nt_store" ? m->nt_store : m->nt_load) = value;
    }
    else if (n == "direct") {
        if (value < 0 || value > 2) return fail(PCD_INVALID_VALUE, "direct must be 0, 1 or 2");
        if (value == 2 && m->dtype == PCD_F32)
            return fail(PCD_INVALID_VALUE, "direct = 2: the direct-weight tile takes 16-bit operands");
        if (value == 2 && m->Wpk.empty())
            if (int st = alloc_direct(m)) return st;
        m->direct = value;
    }
    else if (n == "k_stagger") {
        if (value < kKStaggerAuto || value > kMaxKStagger)
            return fail(PCD_INVALID_VALUE, "k_stagger must be -1 (automatic), 0 (off) or up to %d", kMaxKStagger);
        m->k_stagger = value;
    } else return fail(PCD_INVALID_VALUE, "unknown option '%s'", name);
    // cached graphs were captured with the old options
    return drop_plans(m);
}

int pcd_pc_profile_result(pcd_model* m, float* err_ms, float* upd_ms, int* launches) {
    if (int st = check_model(m)) return st;
    if (err_ms) *err_ms = m->prof_err_ms;
    if (upd_ms) *upd_ms = m->prof_upd_ms;
    if (launches) *launches = m->prof_launches;
    return PCD_SUCCESS;
}

static int copy_out_rows(float* dst, int cols, const float* src, int ld, int rows, hipStream_t s) {
    HIP_TRY(hipMemcpy2DAsync(dst, (size_t)cols * 4, src, (size_t)ld * 4, (size_t)cols * 4, rows,
                             hipMemcpyDeviceToDevice, s));
    return PCD_SUCCESS;
}

// Copies every layer's first `batch` rows, layer after layer, into out_states.
static int copy_out_states(pcd_model* m, Workspace* w, float* out_states, int batch, hipStream_t s) {
    size_t off = 0;
    for (int l = 0; l < m->L; ++l) {
        if (int st = copy_out_rows(out_states + off, m->s[l], w->M[l], m->P[l], batch, s)) return st;
        off += (size_t)batch * m->s[l];
    }
    return PCD_SUCCESS;
}

int pcd_pc_relax(pcd_model* m, const float* x0, int batch, int steps, float* out_top, float* out_states,
                 float* out_energy, void* stream_) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (steps < 1) return fail(PCD_INVALID_VALUE, "inferenceSteps must be >= 1, got %d", steps);
    if (!x0 || !out_top) return fail(PCD_INVALID_VALUE, "pcd_pc_relax: null pointer");
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, batch, &w)) return st;
    const int L = m->L;
    HIP_TRY(hipMemcpy2DAsync(w->M[0], (size_t)m->P[0] * 4, x0, (size_t)m->s[0] * 4, (size_t)m->s[0] * 4, batch,
                             hipMemcpyDeviceToDevice, s));
    const float* energy = nullptr;
    if (int st = run_relax(m, w, batch, steps, 0, out_energy != nullptr, out_energy, s, &energy)) return st;
    if (int st = copy_out_rows(out_top, m->s[L - 1], w->M[L - 1], m->P[L - 1], batch, s)) return st;
    if (out_states)
        if (int st = copy_out_states(m, w, out_states, batch, s)) return st;
    if (out_energy && energy != out_energy)
        HIP_TRY(hipMemcpyAsync(out_energy, energy, (size_t)steps * batch * 4, hipMemcpyDeviceToDevice, s));
    return PCD_SUCCESS;
}

}  // extern "C"

// ------------------------------------------------- allocation-free relaxation

// Scratch of pcd_pc_relax_noalloc: every buffer its settling needs besides the
// caller's inputs and outputs (states, their 16-bit copies, deltas, folded
// updates, energy partials, split-K partial tiles and counters), carved per
// call.  Each device the library runs on holds its own copy of the array
// until the process ends.  In host code the name is a host-side stand-in, not
// a device address: host code uses only the address scratch_device() looks up.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;

// One device's use of the array: its address, and the order of the calls
// that use it.  `mu` is held for the whole of a call's enqueue, so calls from
// several threads (and models) take the array one at a time on the host;
// `done` is recorded on a call's stream after its last launch, and the next
// call's stream waits on it before its first, so calls on different streams
// also run one after another on the device, without any allocation.
struct ScratchDevice {
    std::mutex mu;
    char* base = nullptr;
    hipEvent_t done = nullptr;
    bool recorded = false;
};
std::mutex g_scratch_mu;
ScratchDevice g_scratch[kMaxScratchDevices];

// The scratch record of `device`, which must be current.  Set up on the first
// call for that device: the array's device address from hipGetSymbolAddress
// (each device holds the array at its own address) and the ordering event.
int scratch_device(int device, ScratchDevice** out) {
    if (device < 0 || device >= kMaxScratchDevices)
        return fail(PCD_INVALID_VALUE, "device %d beyond the %d the scratch table covers", device, kMaxScratchDevices);
    std::lock_guard<std::mutex> g(g_scratch_mu);
    ScratchDevice& sd = g_scratch[device];
    if (!sd.base) {
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(PCD_HIP_ERROR, "hipGetSymbolAddress(scratch) gave a null address");
        HIP_TRY(hipEventCreateWithFlags(&sd.done, hipEventDisableTiming));
        sd.base = (char*)p;
    }
    *out = &sd;
    return PCD_SUCCESS;
}

// Lays out the workspace of a `batch`-row settling with `tile` from `base`:
// the buffers ensure_workspace allocates (energy slots for this tile only),
// then split-K scratch for exactly the partial tiles this call's phases use
// (the split plan itself is the allocating path's, so the kernels and their
// results are the same).  Returns the bytes the layout spans.
size_t carve_workspace(const pcd_model* m, char* base, int batch, Tile tile, Workspace& w) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char* p = base + off;
        off += round_up(bytes, 256);
        return p;
    };
    const int L = m->L, ob = op_bytes(m->dtype);
    w.cap = (int)round_up((size_t)batch, kRowPad);
    const size_t cap = (size_t)w.cap;
    w.M.assign(L, nullptr);
    w.S.assign(L, nullptr);
    w.D.assign(L, nullptr);
    w.E.assign(L, nullptr);
    for (int l = 0; l < L; ++l) {
        w.M[l] = (float*)take(cap * m->P[l] * 4);
        if (l >= 1 && m->dtype != PCD_F32) w.S[l] = take(cap * m->P[l] * ob);
        if (l >= 1) w.D[l] = take(cap * m->P[l - 1] * ob);
        if (l >= 1 && l <= L - 2) w.E[l] = (float*)take(cap * m->P[l] * 4);
    }
    w.slots_cap = energy_slots(m, tile);
    w.energy_part = (float*)take((size_t)w.slots_cap * cap * 4);
    w.split_count = (int*)take(split_count_bytes(m));
    w.split_part = (float*)(base + off);
    std::vector<ProblemSet> err, upd;
    int nslots = 0;
    build_phase_sets(m, &w, batch, tile, 0, err, upd, &nslots);
    size_t end = off;
    for (const auto* sets : {&err, &upd})
        for (const ProblemSet& ps : *sets)
            for (int i = 0; i < ps.n; ++i)
                if (ps.p[i].ksplit > 1)
                    end = std::max(end, (size_t)((const char*)(ps.p[i].part + (size_t)ps.p[i].tiles * tile.m * tile.n) -
                                                 base));
    return round_up(end, 256);
}

}  // namespace

extern "C" {

int pcd_pc_relax_noalloc(pcd_model* m, const float* x0, int batch, int steps, float* out_top, float* out_states,
                         float* out_energy, void* stream_) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (steps < 1) return fail(PCD_INVALID_VALUE, "inferenceSteps must be >= 1, got %d", steps);
    if (!x0 || !out_top) return fail(PCD_INVALID_VALUE, "pcd_pc_relax_noalloc: null pointer");
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    ScratchDevice* sd = nullptr;
    if (int st = scratch_device(m->device, &sd)) return st;
    std::lock_guard<std::mutex> dg(sd->mu);
    char* const base = sd->base;
    // Outside graph capture, this call's work starts after the previous call's
    // (on whatever stream) has finished with the array.  A call captured into
    // a graph is ordered by the graph's own stream: the caller orders its
    // replays against other uses of the array.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (!capturing && sd->recorded) HIP_TRY(hipStreamWaitEvent(s, sd->done, 0));
    const Tile tile = choose_tile(m, batch);
    Workspace w;
    w.stream = s;
    const size_t need = carve_workspace(m, base, batch, tile, w);
    if (need > kNoAllocScratchBytes)
        return fail(PCD_INVALID_VALUE,
                    "pcd_pc_relax_noalloc: %d rows of this model need %zu bytes of scratch, beyond its %zu; use "
                    "pcd_pc_relax", batch, need, kNoAllocScratchBytes);
    // The array keeps whatever the last call on this device left in it: clear
    // the whole span (the K padding of the states and deltas and the split-K
    // counters must read zero) with a kernel, which also records into a
    // captured graph.
    if (int st = launch_zero(base, need, s)) return st;
    const int L = m->L;
    HIP_TRY(hipMemcpy2DAsync(w.M[0], (size_t)m->P[0] * 4, x0, (size_t)m->s[0] * 4, (size_t)m->s[0] * 4, batch,
                             hipMemcpyDeviceToDevice, s));
    RelaxSpec r;
    r.batch = batch;
    r.steps = steps;
    r.tile = tile;
    r.energy_out = out_energy;   // [steps x batch], written in place
    if (int st = enqueue_relax(m, &w, r, s, nullptr)) return st;
    if (int st = copy_out_rows(out_top, m->s[L - 1], w.M[L - 1], m->P[L - 1], batch, s)) return st;
    if (out_states)
        if (int st = copy_out_states(m, &w, out_states, batch, s)) return st;
    if (!capturing) {
        HIP_TRY(hipEventRecord(sd->done, s));
        sd->recorded = true;
    }
    return PCD_SUCCESS;
}

int pcd_pc_relax_ragged(pcd_model* m, const float* x0_packed, const int* row_offsets, const int* steps, int requests,
                        int exit_rule, float exit_threshold, int* steps_used, float* out_top, float* out_energy,
                        void* stream_) {
    if (int st = check_model(m)) return st;
    if (requests < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (!x0_packed || !row_offsets || !steps || !steps_used || !out_top)
        return fail(PCD_INVALID_VALUE, "pcd_pc_relax_ragged: null pointer");
    if (exit_rule < PCD_EXIT_NONE || exit_rule > PCD_EXIT_ABSOLUTE)
        return fail(PCD_INVALID_VALUE, "unknown exit rule %d", exit_rule);
    if (row_offsets[0] != 0) return fail(PCD_INVALID_VALUE, "row_offsets[0] must be 0");
    int tmax = 0;
    for (int r = 0; r < requests; ++r) {
        if (row_offsets[r + 1] <= row_offsets[r]) return fail(PCD_INVALID_VALUE, "request %d has no rows", r);
        if (steps[r] < 1) return fail(PCD_INVALID_VALUE, "request %d: steps must be >= 1", r);
        tmax = std::max(tmax, steps[r]);
    }
    const int rows = row_offsets[requests];
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, rows, &w)) return st;
    const int L = m->L;
    const Tile tile = choose_tile(m, rows);
    // Settling order: requests by decreasing step budget (stable).  As
    // requests reach their budgets the rows still running shrink towards a
    // prefix of the packing, and the row tiles past it drop out of the phases
    // whole (the per-step tile list deals only running tiles) instead of
    // staying partly busy.  Option ragged_order = 0 keeps the caller's order.
    // Rows never interact, so fp32 results do not depend on the order.
    std::vector<int> order(requests);
    for (int r = 0; r < requests; ++r) order[r] = r;
    if (m->ragged_order)
        std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return steps[a] > steps[b]; });
    bool identity = true;
    for (int r = 0; r < requests; ++r) identity = identity && order[r] == r;
    // Small per-call tables: rows' request ids, request offsets, step
    // budgets, exit state and (settling order) the caller's row of each
    // settled row.  They live in a workspace buffer sized for the largest call
    // the workspace takes (rows <= cap, requests <= rows), at offsets fixed by
    // (rows, requests), so the cached graph of a loop of the same shape finds
    // this call's tables where it was captured.
    const size_t tbytes = (size_t)rows * 4 + (size_t)(requests + 1) * 4 + (size_t)requests * 4 * 3 + (size_t)rows * 4;
    if (!w->rg_tables) {
        const size_t cap_bytes = (size_t)w->cap * 4 + (size_t)(w->cap + 1) * 4 + (size_t)w->cap * 4 * 3 +
                                 (size_t)w->cap * 4;
        if (int st = dev_alloc_zero(w->owned, &w->rg_tables, cap_bytes)) return st;
    }
    void* tables = w->rg_tables;
    int* d_row_req = (int*)tables;
    int* d_offsets = d_row_req + rows;
    int* d_done = d_offsets + requests + 1;
    float* d_prev = (float*)(d_done + requests);
    float* d_last = d_prev + requests;
    int* d_perm = (int*)(d_last + requests);
    std::vector<char> host(tbytes, 0);
    int* h_row_req = (int*)host.data();
    int* h_offsets = h_row_req + rows;
    int* h_steps = h_offsets + requests + 1;
    int* h_perm = (int*)host.data() + rows + (requests + 1) + 3 * (size_t)requests;
    h_offsets[0] = 0;
    for (int k = 0; k < requests; ++k) {
        const int r = order[k], n = row_offsets[r + 1] - row_offsets[r];
        h_offsets[k + 1] = h_offsets[k] + n;
        h_steps[k] = steps[r];
        for (int i = 0; i < n; ++i) {
            h_row_req[h_offsets[k] + i] = k;
            h_perm[h_offsets[k] + i] = row_offsets[r] + i;
        }
    }
    int st = PCD_SUCCESS;
    hipError_t e = hipMemcpyAsync(tables, host.data(), tbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        if (identity) {
            e = hipMemcpy2DAsync(w->M[0], (size_t)m->P[0] * 4, x0_packed, (size_t)m->s[0] * 4,
                                 (size_t)m->s[0] * 4, rows, hipMemcpyDeviceToDevice, s);
        } else {
            const int grid = (int)std::min<size_t>(((size_t)rows * m->s[0] + 255) / 256, 4096);
            hipLaunchKernelGGL(permute_rows_kernel, dim3(grid), dim3(256), 0, s, x0_packed, m->s[0], w->M[0],
                               m->P[0], (const int*)d_perm, rows, m->s[0], 1);
            e = hipGetLastError();
        }
    }
    if (e != hipSuccess) st = from_hip(e, "ragged upload");
    if (!st) {
        RelaxSpec r;
        r.batch = rows;
        r.steps = tmax;
        r.tile = tile;
        r.row_req = d_row_req;
        r.done_at = d_done;
        r.row_offsets = d_offsets;
        r.requests = requests;
        r.exit_rule = exit_rule;
        r.exit_thr = exit_threshold;
        r.prev_energy = d_prev;
        r.last_energy = d_last;
        if (m->profile || !m->use_graph) {
            // With the profile option, every phase launch is timed (eagerly).
            PhaseTimer timer;
            st = enqueue_relax(m, w, r, s, m->profile ? &timer : nullptr);
            if (m->profile) {
                int st2 = collect_timer(m, timer, s);
                if (!st) st = st2;
            }
        } else {
            // The loop of tmax steps as one graph: requests that have exited
            // keep their states, and steps after every request has exited
            // find no running row tile and return at once.
            Plan* p = get_plan(m, w, r, 0, &st);
            if (p) {
                e = hipGraphLaunch(p->exec, s);
                if (e != hipSuccess) st = from_hip(e, "hipGraphLaunch");
            }
        }
    }
    if (!st) {
        if (identity) {
            st = copy_out_rows(out_top, m->s[L - 1], w->M[L - 1], m->P[L - 1], rows, s);
        } else {
            const int grid = (int)std::min<size_t>(((size_t)rows * m->s[L - 1] + 255) / 256, 4096);
            hipLaunchKernelGGL(permute_rows_kernel, dim3(grid), dim3(256), 0, s, (const float*)w->M[L - 1],
                               m->P[L - 1], out_top, m->s[L - 1], (const int*)d_perm, rows, m->s[L - 1], 0);
            st = from_hip(hipGetLastError(), "permute_rows_kernel launch");
        }
    }
    std::vector<int> used(requests);
    std::vector<float> last(requests);
    if (!st) {
        e = hipMemcpyAsync(used.data(), d_done, (size_t)requests * 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipMemcpyAsync(last.data(), d_last, (size_t)requests * 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) st = from_hip(e, "ragged download");
    }
    if (!st) {
        for (int k = 0; k < requests; ++k) {
            steps_used[order[k]] = used[k];
            if (out_energy) out_energy[order[k]] = last[k];
        }
    }
    if (st) (void)hipStreamSynchronize(s);   // the upload reads `host` until the stream reaches it
    return st;
}

// ------------------------------------------- clamped settling, classes, learning

// Writes rows of layer lt's state (and its operand-type copy) before a
// settling: src [rows x s_lt] packed, or, with src null, the one-hot label of
// class r % s_lt for row r.  Columns past s_lt are written zero.
static int stage_rows(pcd_model* m, Workspace* w, int lt, const float* src, int rows, hipStream_t s) {
    const size_t n = (size_t)rows * m->P[lt];
    const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
    switch (m->dtype) {
    case PCD_F32:
        hipLaunchKernelGGL(top_rows_kernel<float>, dim3(grid), dim3(256), 0, s, src, m->s[lt], rows, w->M[lt],
                           nullptr, m->P[lt]);
        break;
    case PCD_BF16:
        hipLaunchKernelGGL(top_rows_kernel<bf16_t>, dim3(grid), dim3(256), 0, s, src, m->s[lt], rows, w->M[lt],
                           w->S[lt], m->P[lt]);
        break;
    default:
        hipLaunchKernelGGL(top_rows_kernel<f16_t>, dim3(grid), dim3(256), 0, s, src, m->s[lt], rows, w->M[lt],
                           w->S[lt], m->P[lt]);
        break;
    }
    return from_hip(hipGetLastError(), "top_rows_kernel launch");
}

// The clamped top rows of a settling (see stage_rows).
static int stage_top(pcd_model* m, Workspace* w, const float* src, int rows, hipStream_t s) {
    return stage_rows(m, w, m->L - 1, src, rows, s);
}

// After the fp32 weights of layer l changed (the fp32 W itself, or a 16-bit
// model's masters W32): W^T, and for 16-bit models W, re-derived in the
// operand type (rounded to nearest even).
static int refresh_operands(pcd_model* m, int l, hipStream_t s) {
    const int lo = m->s[l - 1], sz = m->s[l];
    const int Rlo = (int)round_up(lo, kRowPad), Rsz = (int)round_up(sz, kRowPad);
    const void* src = m->dtype == PCD_F32 ? (const void*)m->W[l] : (const void*)m->W32[l];
    switch (m->dtype) {
    case PCD_F32:
        pack_op<float>(s, src, 1, m->P[l], lo, 1, m->WT[l], Rsz,
                           m->P[l - 1], m->P[l - 1]);
        break;
    case PCD_BF16:
        pack_op<bf16_t>(s, src, 1, Rlo, m->P[l], 0, m->W[l], Rlo,
                           m->P[l], m->P[l]);
        pack_op<bf16_t>(s, src, 1, m->P[l], lo, 1, m->WT[l], Rsz,
                           m->P[l - 1], m->P[l - 1]);
        break;
    default:
        pack_op<f16_t>(s, src, 1, Rlo, m->P[l], 0, m->W[l], Rlo,
                           m->P[l], m->P[l]);
        pack_op<f16_t>(s, src, 1, m->P[l], lo, 1, m->WT[l], Rsz,
                           m->P[l - 1], m->P[l - 1]);
        break;
    }
    if (int st = from_hip(hipGetLastError(), "operand refresh")) return st;
    return repack_direct(m, l, s);
}

int pcd_pc_relax_clamped(pcd_model* m, const float* x0, const float* top, int batch, int steps, float* out_states,
                         float* out_energy, void* stream_) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (steps < 1) return fail(PCD_INVALID_VALUE, "inferenceSteps must be >= 1, got %d", steps);
    if (!x0 || !top) return fail(PCD_INVALID_VALUE, "pcd_pc_relax_clamped: null pointer");
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, batch, &w)) return st;
    HIP_TRY(hipMemcpy2DAsync(w->M[0], (size_t)m->P[0] * 4, x0, (size_t)m->s[0] * 4, (size_t)m->s[0] * 4, batch,
                             hipMemcpyDeviceToDevice, s));
    if (int st = stage_top(m, w, top, batch, s)) return st;
    const float* energy = nullptr;
    if (int st = run_relax(m, w, batch, steps, 1, out_energy != nullptr, out_energy, s, &energy)) return st;
    if (out_states)
        if (int st = copy_out_states(m, w, out_states, batch, s)) return st;
    if (out_energy && energy != out_energy)
        HIP_TRY(hipMemcpyAsync(out_energy, energy, (size_t)steps * batch * 4, hipMemcpyDeviceToDevice, s));
    return PCD_SUCCESS;
}

int pcd_pc_classify(pcd_model* m, const float* x0, int batch, int steps, float* out_class_energies, int* out_class,
                    float* out_energy, void* stream_) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (steps < 1) return fail(PCD_INVALID_VALUE, "inferenceSteps must be >= 1, got %d", steps);
    if (!x0) return fail(PCD_INVALID_VALUE, "pcd_pc_classify: null input");
    if (!out_class_energies && !out_class && !out_energy)
        return fail(PCD_INVALID_VALUE, "pcd_pc_classify: no output requested");
    const int C = m->s[m->L - 1];
    const long rows_l = (long)batch * C;
    if (rows_l > (1L << 30)) return fail(PCD_INVALID_VALUE, "pcd_pc_classify: %d x %d rows is too many", batch, C);
    const int rows = (int)rows_l;
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, rows, &w)) return st;
    {
        const size_t n = (size_t)rows * m->s[0];
        const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
        hipLaunchKernelGGL(replicate_rows_kernel, dim3(grid), dim3(256), 0, s, x0, m->s[0], C, rows, w->M[0],
                           m->P[0]);
        if (int st = from_hip(hipGetLastError(), "replicate_rows_kernel launch")) return st;
    }
    if (int st = stage_top(m, w, nullptr, rows, s)) return st;
    // Eager runs write the energies into a stream-ordered scratch buffer.
    void* energy_buf = nullptr;
    if (m->profile || !m->use_graph)
        if (int st = pool_alloc(&energy_buf, (size_t)steps * rows * 4, s)) return st;
    const float* energy = nullptr;
    int st = run_relax(m, w, rows, steps, 1, 1, (float*)energy_buf, s, &energy);
    if (!st) {
        const int grid = std::min((batch + 255) / 256, 1024);
        hipLaunchKernelGGL(class_argmin_kernel, dim3(grid), dim3(256), 0, s, energy + (size_t)(steps - 1) * rows,
                           batch, C, out_class_energies, out_class, out_energy);
        st = from_hip(hipGetLastError(), "class_argmin_kernel launch");
    }
    if (energy_buf) {
        int st2 = pool_free(energy_buf, s);
        if (!st) st = st2;
    }
    return st;
}

int pcd_pc_classify_adaptive(pcd_model* m, const float* x0, int batch, int max_steps, float epsilon,
                             float* out_class_energies, int* out_class_steps, int* out_class, float* out_energy,
                             int* out_steps_used, void* stream_) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (max_steps < 1) return fail(PCD_INVALID_VALUE, "maxSteps must be >= 1, got %d", max_steps);
    if (!x0) return fail(PCD_INVALID_VALUE, "pcd_pc_classify_adaptive: null input");
    if (!out_class_energies && !out_class_steps && !out_class && !out_energy && !out_steps_used)
        return fail(PCD_INVALID_VALUE, "pcd_pc_classify_adaptive: no output requested");
    const int C = m->s[m->L - 1];
    const long rows_l = (long)batch * C;
    if (rows_l > (1L << 30))
        return fail(PCD_INVALID_VALUE, "pcd_pc_classify_adaptive: %d x %d rows is too many", batch, C);
    const int rows = (int)rows_l;
    hipStream_t s = (hipStream_t)stream_;
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, rows, &w)) return st;
    // Candidate c of sample b is row b * C + c (SettleCandidate, Network.cs:851-867):
    // layer 0 its sample, the top one-hot(c), the hidden layers from zero.
    {
        const size_t n = (size_t)rows * m->s[0];
        const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
        hipLaunchKernelGGL(replicate_rows_kernel, dim3(grid), dim3(256), 0, s, x0, m->s[0], C, rows, w->M[0],
                           m->P[0]);
        if (int st = from_hip(hipGetLastError(), "replicate_rows_kernel launch")) return st;
    }
    if (int st = stage_top(m, w, nullptr, rows, s)) return st;
    // Every candidate is a request of one row that leaves by the relative rule
    // (SettleAdaptive, :876-907).  The tables take the ragged layout in the
    // workspace buffer (offsets fixed by rows and requests, which a cached
    // graph relies on), written on the device.
    if (!w->rg_tables) {
        const size_t cap_bytes = (size_t)w->cap * 4 + (size_t)(w->cap + 1) * 4 + (size_t)w->cap * 4 * 3 +
                                 (size_t)w->cap * 4;
        if (int st = dev_alloc_zero(w->owned, &w->rg_tables, cap_bytes)) return st;
    }
    int* d_row_req = (int*)w->rg_tables;
    int* d_offsets = d_row_req + rows;
    int* d_done = d_offsets + rows + 1;
    float* d_prev = (float*)(d_done + rows);
    float* d_last = d_prev + rows;
    {
        const int grid = std::min((rows + 256) / 256, 4096);
        hipLaunchKernelGGL(row_request_tables_kernel, dim3(grid), dim3(256), 0, s, d_row_req, d_offsets, d_done,
                           d_prev, d_last, rows, max_steps);
        if (int st = from_hip(hipGetLastError(), "row_request_tables_kernel launch")) return st;
    }
    RelaxSpec r;
    r.batch = rows;
    r.steps = max_steps;
    r.tile = choose_tile(m, rows);
    r.clamp_top = 1;
    r.row_req = d_row_req;
    r.done_at = d_done;
    r.row_offsets = d_offsets;
    r.requests = rows;
    r.exit_rule = PCD_EXIT_RELATIVE;
    r.exit_thr = epsilon;
    r.prev_energy = d_prev;
    r.last_energy = d_last;
    int st = PCD_SUCCESS;
    if (m->profile || !m->use_graph) {
        PhaseTimer timer;
        st = enqueue_relax(m, w, r, s, m->profile ? &timer : nullptr);
        if (m->profile) {
            int st2 = collect_timer(m, timer, s);
            if (!st) st = st2;
        }
    } else {
        Plan* p = get_plan(m, w, r, 0, &st);
        if (p) st = from_hip(hipGraphLaunch(p->exec, s), "hipGraphLaunch");
    }
    if (st) return st;
    const int grid = std::min((batch + 255) / 256, 1024);
    hipLaunchKernelGGL(adaptive_argmin_kernel, dim3(grid), dim3(256), 0, s, (const float*)d_last, (const int*)d_done,
                       batch, C, out_class_energies, out_class_steps, out_class, out_energy, out_steps_used);
    return from_hip(hipGetLastError(), "adaptive_argmin_kernel launch");
}

}  // extern "C"

// The learning step (pcd_pc_learn, pcd_pc_learn_warm): settle from hidden_in
// (null: zero hidden states), hand the settled hidden states to hidden_out
// (nullable), then update every layer's weights.
static int learn_step(pcd_model* m, const float* x0, const float* labels, const float* hidden_in, float* hidden_out,
                      int batch, int steps, float eta_w, float weight_decay, float* out_energy, hipStream_t s) {
    if (int st = check_model(m)) return st;
    if (batch < 1) return fail(PCD_INVALID_VALUE, "Empty batch.");
    if (steps < 1) return fail(PCD_INVALID_VALUE, "inferenceSteps must be >= 1, got %d", steps);
    if (!x0 || !labels) return fail(PCD_INVALID_VALUE, "pcd_pc_learn: null pointer");
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    Workspace* w = nullptr;
    if (int st = ensure_workspace(m, s, batch, &w)) return st;
    const int L = m->L;
    HIP_TRY(hipMemcpy2DAsync(w->M[0], (size_t)m->P[0] * 4, x0, (size_t)m->s[0] * 4, (size_t)m->s[0] * 4, batch,
                             hipMemcpyDeviceToDevice, s));
    if (int st = stage_top(m, w, labels, batch, s)) return st;
    const bool warm = hidden_in != nullptr && L > 2;
    if (warm) {
        size_t off = 0;
        for (int l = 1; l <= L - 2; ++l) {
            if (int st = stage_rows(m, w, l, hidden_in + off, batch, s)) return st;
            off += (size_t)batch * m->s[l];
        }
    }
    void* energy_buf = nullptr;
    const bool want_energy = out_energy != nullptr;
    if (want_energy && (m->profile || !m->use_graph))
        if (int st = pool_alloc(&energy_buf, (size_t)steps * batch * 4, s)) return st;
    const float* energy = nullptr;
    int st = run_relax(m, w, batch, steps, 1, want_energy, (float*)energy_buf, s, &energy, warm ? 1 : 0);
    if (!st && want_energy) {
        hipError_t e = hipMemcpyAsync(out_energy, energy + (size_t)(steps - 1) * batch, (size_t)batch * 4,
                                      hipMemcpyDeviceToDevice, s);
        st = from_hip(e, "learn energy copy");
    }
    if (!st && hidden_out) {
        size_t off = 0;
        for (int l = 1; l <= L - 2 && !st; ++l) {
            st = copy_out_rows(hidden_out + off, m->s[l], w->M[l], m->P[l], batch, s);
            off += (size_t)batch * m->s[l];
        }
    }

    // Hebbian step of every layer (Layer.UpdateWeights, Layer.cs:320-333):
    // W_l = (1 - eta_w lambda) (W_l + eta_w D_l^T M_l), the bias sums, and the
    // operand copies the settling reads (W_l^T; W_l for 16-bit models).
    const float keep = 1.f - eta_w * weight_decay;
    if (!st && batch <= kHebbValuRows) {
        // At most kHebbValuRows rows: one launch of hebbian_small_kernel.
        for (int l0 = 1; l0 < L && !st; l0 += kHebbLayers) {
            HebbSet hs;
            std::memset(&hs, 0, sizeof hs);
            hs.batch = batch;
            hs.alpha = eta_w * keep;
            hs.beta = keep;
            hs.eta_w = eta_w;
            int blocks = 0;
            for (int l = l0; l < L && hs.n < kHebbLayers; ++l) {
                HebbLayer& h = hs.l[hs.n++];
                h.d = w->D[l];
                h.ldd = m->P[l - 1];
                h.m = w->M[l];
                h.ldm = m->P[l];
                h.w = m->dtype == PCD_F32 ? (float*)m->W[l] : m->W32[l];
                h.w16 = m->dtype == PCD_F32 ? nullptr : m->W[l];
                h.ldw = m->P[l];
                h.wt = m->WT[l];
                h.ldwt = m->P[l - 1];
                h.bias = m->bias[l];
                h.lo = m->s[l - 1];
                h.sz = m->s[l];
                h.blocks = ((h.lo + 31) / 32) * ((h.sz + 31) / 32);
                blocks += h.blocks;
            }
            switch (m->dtype) {
            case PCD_F32: hipLaunchKernelGGL(hebbian_small_kernel<float>, dim3(blocks), dim3(256), 0, s, hs); break;
            case PCD_BF16: hipLaunchKernelGGL(hebbian_small_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, hs); break;
            default: hipLaunchKernelGGL(hebbian_small_kernel<f16_t>, dim3(blocks), dim3(256), 0, s, hs); break;
            }
            st = from_hip(hipGetLastError(), "hebbian_small_kernel launch");
            for (int l = l0; l < std::min(L, l0 + kHebbLayers) && !st; ++l) st = repack_direct(m, l, s);
        }
        if (energy_buf) {
            int st2 = pool_free(energy_buf, s);
            if (!st) st = st2;
        }
        return st;
    }
    // A larger batch: one grouped GEMM over the batch (K = rows; D_l and M_l
    // transposed so K is contiguous), the bias sums, then the refreshed copies.
    const int kp = (int)round_up((size_t)batch, kFeatPad);
    std::vector<void*> tmp;
    std::vector<ProblemSet> sets;
    const Tile tile = Tile{64, 64};
    for (int l = 1; l < L && !st; ++l) {
        const int lo = m->s[l - 1], sz = m->s[l];
        const int Rlo = (int)round_up(lo, kRowPad), Rsz = (int)round_up(sz, kRowPad);
        void *dt = nullptr, *mt = nullptr;
        if ((st = pool_alloc(&dt, (size_t)Rlo * kp * 4, s))) break;
        tmp.push_back(dt);
        if ((st = pool_alloc(&mt, (size_t)Rsz * kp * 4, s))) break;
        tmp.push_back(mt);
        const int g1 = (int)std::min<size_t>(((size_t)Rlo * kp + 255) / 256, 8192);
        const int gb = std::min((lo + 255) / 256, 1024);
        // D_l^T (D is in the operand type: a 16-bit model's update uses the
        // rounded Delta its settling's W^T GEMM consumed), M_l^T, and the bias
        switch (m->dtype) {
        case PCD_F32:
            pack_op<float>(s, (const void*)w->D[l], 1, m->P[l - 1],
                               batch, 1, dt, Rlo, kp, kp);
            hipLaunchKernelGGL(bias_update_kernel<float>, dim3(gb), dim3(256), 0, s, (const void*)w->D[l],
                               m->P[l - 1], batch, lo, m->bias[l], eta_w);
            break;
        case PCD_BF16:
            hipLaunchKernelGGL(pack_record_kernel<float>, dim3(g1), dim3(256), 0, s, (const void*)w->D[l],
                               (int)REC_BF16, nullptr, nullptr, m->P[l - 1], batch, 1, dt, Rlo, kp);
            hipLaunchKernelGGL(bias_update_kernel<bf16_t>, dim3(gb), dim3(256), 0, s, (const void*)w->D[l],
                               m->P[l - 1], batch, lo, m->bias[l], eta_w);
            break;
        default:
            hipLaunchKernelGGL(pack_record_kernel<float>, dim3(g1), dim3(256), 0, s, (const void*)w->D[l],
                               (int)REC_F16, nullptr, nullptr, m->P[l - 1], batch, 1, dt, Rlo, kp);
            hipLaunchKernelGGL(bias_update_kernel<f16_t>, dim3(gb), dim3(256), 0, s, (const void*)w->D[l],
                               m->P[l - 1], batch, lo, m->bias[l], eta_w);
            break;
        }
        pack_op<float>(s, (const void*)w->M[l], 1, m->P[l], batch, 1,
                           mt, Rsz, kp, kp);
        if ((st = from_hip(hipGetLastError(), "learning-step packing"))) break;
        if (sets.empty() || sets.back().n == kMaxProblems) {
            sets.emplace_back();
            std::memset(&sets.back(), 0, sizeof(ProblemSet));
        }
        Problem& p = sets.back().p[sets.back().n++];
        p.A = dt;
        p.lda = kp;
        p.B = mt;
        p.ldb = kp;
        p.M = lo;
        p.N = sz;
        p.K = kp;
        p.tiles_m = (lo + tile.m - 1) / tile.m;
        p.tiles_n = (sz + tile.n - 1) / tile.n;
        p.tiles = p.tiles_m * p.tiles_n;
        p.ldo = m->P[l];
        p.m = m->dtype == PCD_F32 ? (float*)m->W[l] : m->W32[l];   // fp32 weights or masters
    }
    if (!st) {
        PhaseArgs a;
        std::memset(&a, 0, sizeof a);
        a.alpha = eta_w * keep;
        a.beta = keep;
        a.tile_order = m->tile_order;
        for (auto& ps : sets)
            if ((st = launch_phase(PCD_F32, tile, EPI_PLAIN, ps, a, s))) break;
    }
    for (int l = 1; l < L && !st; ++l) st = refresh_operands(m, l, s);
    for (void* t : tmp) {
        int st2 = pool_free(t, s);
        if (!st) st = st2;
    }
    if (energy_buf) {
        int st2 = pool_free(energy_buf, s);
        if (!st) st = st2;
    }
    return st;
}

extern "C" {

int pcd_pc_learn(pcd_model* m, const float* x0, const float* labels, int batch, int steps, float eta_w,
                 float weight_decay, float* out_energy, void* stream) {
    return learn_step(m, x0, labels, nullptr, nullptr, batch, steps, eta_w, weight_decay, out_energy,
                      (hipStream_t)stream);
}

int pcd_pc_learn_warm(pcd_model* m, const float* x0, const float* labels, const float* hidden_in, float* hidden_out,
                      int batch, int steps, float eta_w, float weight_decay, float* out_energy, void* stream) {
    return learn_step(m, x0, labels, hidden_in, hidden_out, batch, steps, eta_w, weight_decay, out_energy,
                      (hipStream_t)stream);
}

int pcd_pc_model_get_weights(pcd_model* m, int layer, float* W_out, float* b_out) {
    if (int st = check_model(m)) return st;
    if (layer < 1 || layer >= m->L) return fail(PCD_INVALID_VALUE, "layer %d is not in 1..%d", layer, m->L - 1);
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(device_sync());
    const int lo = m->s[layer - 1], sz = m->s[layer];
    if (W_out) {
        const void* src = m->dtype == PCD_F32 ? (const void*)m->W[layer] : (const void*)m->W32[layer];
        HIP_TRY(hipMemcpy2D(W_out, (size_t)sz * 4, src, (size_t)m->P[layer] * 4, (size_t)sz * 4, lo,
                            hipMemcpyDeviceToHost));
    }
    if (b_out) HIP_TRY(sync_memcpy(b_out, m->bias[layer], (size_t)lo * 4, hipMemcpyDeviceToHost));
    return PCD_SUCCESS;
}

// ------------------------------------------------------------ weight records

// A LayerSerializer record (Model/LayerSerializer.cs:8-41): its header and
// where its weights and bias sit.  Mu, PredictionError, PreActivation and
// Prediction are a settling's state, which the device path makes itself.
struct LayerRecord {
    int size = 0, lower = 0, flags = 0, kind = REC_F32;
    float precision = 0.f;
    const uint8_t* weights = nullptr;   // payload in the stored format
    size_t weight_bytes = 0;
    const uint8_t* bias = nullptr;      // [lower] fp32
};

static int parse_record(const void* data, size_t bytes, LayerRecord* r) {
    const uint8_t* p = (const uint8_t*)data;
    const size_t header = 28;   // FixedHeaderBytes, :45
    if (bytes < header) return fail(PCD_INVALID_VALUE, "layer record: %zu bytes is shorter than its header", bytes);
    auto i32 = [&](size_t off) { int32_t v; std::memcpy(&v, p + off, 4); return v; };   // little-endian host
    r->size = i32(0);
    r->lower = i32(4);
    std::memcpy(&r->precision, p + 8, 4);
    r->flags = p[25];
    if (r->size < 1 || r->lower < 0) return fail(PCD_INVALID_VALUE, "layer record: sizes (%d,%d)", r->size, r->lower);
    if (r->flags & 3)
        return fail(PCD_NOT_SUPPORTED, "layer record has a diagonal precision or a prior mean, which the "
                                       "generative snapshot does not carry");
    const int fmt = r->flags & (4 | 8 | 16);
    if (fmt != 0 && fmt != 4 && fmt != 8 && fmt != 16)
        return fail(PCD_INVALID_VALUE, "layer record: more than one weight format flag (0x%x)", r->flags);
    r->kind = fmt == 4 ? REC_F16 : fmt == 8 ? REC_BF16 : fmt == 16 ? REC_I8 : REC_F32;
    const size_t lo = (size_t)r->lower, sz = (size_t)r->size;
    size_t n = header + sz * 8;   // Mu + PredictionError
    if (lo > 0) {
        r->weights = p + n;
        r->weight_bytes = r->kind == REC_F32 ? lo * sz * 4 : r->kind == REC_I8 ? lo * 4 + lo + lo * sz : lo * sz * 2;
        n += r->weight_bytes;
        r->bias = p + n;
        n += lo * 4 * 3;          // Bias, PreActivation, Prediction
    }
    if (bytes != n) return fail(PCD_INVALID_VALUE, "layer record: %zu bytes, the header implies %zu", bytes, n);
    return PCD_SUCCESS;
}

// Weights (W_l and W_l^T in the operand type) and bias of layer `layer` from
// a parsed record.
static hipError_t upload_record_weights(pcd_model* m, int layer, const LayerRecord& r) {
    const int lo = m->s[layer - 1], sz = m->s[layer];
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, r.weight_bytes);
    if (e != hipSuccess) return e;
    e = sync_memcpy(tmp, r.weights, r.weight_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = sync_memcpy(m->bias[layer], r.bias, (size_t)lo * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        const float* scales = r.kind == REC_I8 ? (const float*)tmp : nullptr;
        const int8_t* zeros = r.kind == REC_I8 ? (const int8_t*)tmp + (size_t)lo * 4 : nullptr;
        const void* codes = r.kind == REC_I8 ? (const void*)((const int8_t*)tmp + (size_t)lo * 5) : tmp;
        const int Rlo = (int)round_up(lo, kRowPad), Rsz = (int)round_up(sz, kRowPad);
        const int g1 = (int)std::min<size_t>(((size_t)Rlo * m->P[layer] + 255) / 256, 8192);
        const int g2 = (int)std::min<size_t>(((size_t)Rsz * m->P[layer - 1] + 255) / 256, 8192);
        // W_l as stored ([lo x sz] -> [Rlo x P_l]) and transposed ([sz x lo] -> [Rsz x P_{l-1}]).
        switch (m->dtype) {
        case PCD_F32:
            hipLaunchKernelGGL(pack_record_kernel<float>, dim3(g1), dim3(256), 0, 0, codes, r.kind, scales, zeros, lo,
                               sz, 0, m->W[layer], Rlo, m->P[layer]);
            hipLaunchKernelGGL(pack_record_kernel<float>, dim3(g2), dim3(256), 0, 0, codes, r.kind, scales, zeros, sz,
                               lo, 1, m->WT[layer], Rsz, m->P[layer - 1]);
            break;
        case PCD_BF16:
            hipLaunchKernelGGL(pack_record_kernel<bf16_t>, dim3(g1), dim3(256), 0, 0, codes, r.kind, scales, zeros, lo,
                               sz, 0, m->W[layer], Rlo, m->P[layer]);
            hipLaunchKernelGGL(pack_record_kernel<bf16_t>, dim3(g2), dim3(256), 0, 0, codes, r.kind, scales, zeros, sz,
                               lo, 1, m->WT[layer], Rsz, m->P[layer - 1]);
            break;
        default:
            hipLaunchKernelGGL(pack_record_kernel<f16_t>, dim3(g1), dim3(256), 0, 0, codes, r.kind, scales, zeros, lo,
                               sz, 0, m->W[layer], Rlo, m->P[layer]);
            hipLaunchKernelGGL(pack_record_kernel<f16_t>, dim3(g2), dim3(256), 0, 0, codes, r.kind, scales, zeros, sz,
                               lo, 1, m->WT[layer], Rsz, m->P[layer - 1]);
            break;
        }
        if (m->W32[layer])
            hipLaunchKernelGGL(pack_record_kernel<float>, dim3(g1), dim3(256), 0, 0, codes, r.kind, scales, zeros, lo,
                               sz, 0, m->W32[layer], Rlo, m->P[layer]);
        e = hipGetLastError();
        if (e == hipSuccess && repack_direct(m, layer, 0) != PCD_SUCCESS) e = hipErrorLaunchFailure;
        if (e == hipSuccess) e = device_sync();
    }
    (void)hipFree(tmp);
    return e;
}

int pcd_pc_model_load_record(pcd_model* m, int layer, const void* record, size_t bytes) {
    if (int st = check_model(m)) return st;
    if (!record) return fail(PCD_INVALID_VALUE, "pcd_pc_model_load_record: null record");
    if (layer < 0 || layer >= m->L) return fail(PCD_INVALID_VALUE, "layer %d is not in 0..%d", layer, m->L - 1);
    LayerRecord r;
    if (int st = parse_record(record, bytes, &r)) return st;
    const int lo = layer ? m->s[layer - 1] : 0, sz = m->s[layer];
    if (r.size != sz || r.lower != lo)
        return fail(PCD_INVALID_VALUE, "Layer size mismatch: stored (%d,%d) vs target (%d,%d).", r.size, r.lower, sz, lo);
    if (!(r.precision > 0.f)) return fail(PCD_INVALID_VALUE, "layer record: precision %g is not positive", r.precision);
    std::lock_guard<std::mutex> g(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(device_sync());   // no settling may read the weights while they change
    hipError_t e = hipSuccess;
    if (layer > 0) e = upload_record_weights(m, layer, r);
    if (e != hipSuccess) return from_hip(e, "pcd_pc_model_load_record");
    m->prec[layer] = r.precision;
    // cached graphs carry the precisions in their launch arguments
    return drop_plans(m);
}


}  // extern "C"
