// pc_kernels.hpp -- gfx950 kernels of the batched predictive-coding relaxation.
//
// One relaxation step of BatchedPcForward.cs:93-128 is two grouped launches:
//
//   error phase   for every layer l = 1..L-1 at once (independent problems):
//                   PRE  = S_l . W_l^T           MFMA GEMM [B x s_{l-1}], K = s_l
//                   pred = f(PRE + b_l)
//                   e    = P_{l-1} (M_{l-1} - pred)
//                   d    = f'(PRE + b_l) * e                -> D_l (operand type)
//                   X    = M_{l-1} - eta (e + lambda sign(M_{l-1}))  -> X_{l-1} (fp32)
//                   energy partial 0.5 e^2 / P_{l-1}, summed per row
//   update phase  for every layer l = 1..L-1 at once:
//                   G    = D_l . W_l                 MFMA GEMM [B x s_l], K = s_{l-1}
//                   M_l  = X_l + eta G   (top layer, E = 0: M_l -= eta (lambda sign(M_l) - G))
//                   S_l  = operand-type copy of M_l
// which is the reference's M_l -= eta (E_l - G + lambda sign(M_l)) with the
// terms known before the GEMM folded into X by the phase that has M_l at hand.
//
// Both GEMMs read their operands K-contiguous ("A . B^T" with A [rows x K] and
// B [N x K] row-major): the error phase uses W_l as stored ([s_{l-1} x s_l]),
// the update phase a transposed copy W_l^T ([s_l x s_{l-1}]) made once at
// model upload (the reference transposes every call, BatchedPcForward.cs:62-64).
// The two phases are the Jacobi order of Network.cs:91-110: every error is
// computed from the pre-step states before any state moves.
//
// Tiling: a workgroup owns a BM x BN output tile; its waves (2 x 2, or 2 x 4
// for 256 x 256) each own a (BM/WM) x (BN/WN) part as 32 x 32 MFMA blocks.
// K advances in stages of 64 or 128 bytes per row, copied global -> LDS
// directly (no register staging) a few stages ahead, one barrier per stage;
// 16-byte units are XOR-swizzled by row so that the 16-byte fragment reads of
// a wave hit distinct banks.  The fragment reads of the next 32-byte chunk
// are interleaved with the MFMAs of the current one.  The epilogues keep the
// operands of the next few 32 x 32 blocks in flight while a block computes.
//   16-bit operands: v_mfma_f32_32x32x16_{bf16,f16}; lane l holds 8 consecutive
//     K values of row (l % 32), half-wave l/32 takes the second 8 of each 16.
//   fp32 operands:   v_mfma_f32_32x32x2f32 x 4 per 32-byte chunk: lane l holds 4
//     consecutive floats of row (l % 32); MFMA s uses float s of every lane,
//     so one MFMA sums K indices {c*8+s, c*8+4+s}.
// Result layout (32x32 blocks): register r of lane l is
//   row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

// Lambdas inside kernels must inline, or arrays they touch (the MFMA
// accumulators) lose their registers to the closure's memory.
#define PCD_INLINE __attribute__((always_inline))

namespace pcd {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Keeps
// accumulator indices constant however large the body, where #pragma unroll
// is only a request the unroller may decline.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

enum Act { ACT_LINEAR = 0, ACT_TANH = 1, ACT_RELU = 2, ACT_SIGMOID = 3, ACT_GELU = 4 };
// EPI_PLAIN_KN: the plain product with the B operand row-major [K x N] (the
// layout of Gemm.MatMul's B), read where it lies: each stage's K rows of the
// tile's columns go into LDS as they are and the MFMA fragments come out of
// them through gfx950's transposing LDS read (ds_read_b64_tr_b16), so the
// operand is never packed.  EPI_PLAIN_MK: the same for an A stored [K x M]
// (a transposed A); EPI_PLAIN_MKKN: both.  16-bit operands, LDS-operand tiles.
enum Epi { EPI_ERROR = 0, EPI_UPDATE = 1, EPI_FFG = 2, EPI_PLAIN = 3, EPI_PLAIN_KN = 4, EPI_PLAIN_MK = 5,
           EPI_PLAIN_MKKN = 6 };

// Global-memory accessors.  The epilogue pointers arrive through the
// kernel-argument struct as generic pointers; accessing them through the
// global address space gives global_load/global_store instead of flat ones
// (which also count against the LDS wait counter).
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) uint16_t gu16;
typedef __attribute__((address_space(1))) int gint;
typedef __attribute__((address_space(1))) unsigned long long gu64;
__device__ __forceinline__ float gld(const float* p) { return *(const gfloat*)p; }
__device__ __forceinline__ int gld(const int* p) { return *(const gint*)p; }
__device__ __forceinline__ void gst(float* p, float v) { *(gfloat*)p = v; }
__device__ __forceinline__ void gst(uint16_t* p, uint16_t v) { *(gu16*)p = v; }
// Four consecutive elements in one access (16 bytes of fp32, 8 of a 16-bit type).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) f32x4 gf32x4;
typedef __attribute__((address_space(1))) u32x2 gu32x2;
__device__ __forceinline__ f32x4 gld4(const float* p) { return *(const gf32x4*)p; }
__device__ __forceinline__ void gst4(float* p, f32x4 v) { *(gf32x4*)p = v; }
__device__ __forceinline__ void gst4(uint16_t* p, u32x2 v) { *(gu32x2*)p = v; }

// bf16 and fp16 are carried as raw 16-bit patterns.
struct bf16_t { uint16_t v; };
struct f16_t { uint16_t v; };

// One GEMM of a grouped launch plus the operands of its epilogue.
struct Problem {
    const void* A;        // [>= tiles_m*BM rows x lda], K-contiguous
    const void* B;        // [>= tiles_n*BN rows x ldb], K-contiguous (EPI_PLAIN_KN: [K rows x ldb], N-contiguous)
    int lda, ldb;         // leading dimensions, elements
    int M, N, K;          // valid rows, valid columns, K (a multiple of the stage depth)
    int tiles_m, tiles_n;  // tile grid of the output
    int tiles;            // work units: tiles_m * tiles_n * ksplit
    int ldo;              // leading dimension of every [rows x N] epilogue operand
    const float* bias;    // ERROR/FFG: b_l [N]
    const float* mlow;    // ERROR: fp32 state M_{l-1}
    float* eout;          // ERROR: X_{l-1} = M - eta (E + lambda sign M) (nullable: layer 0 is never updated)
    void* dout;           // ERROR: D_l in the operand type; FFG: operand-type state copy
    float* m;             // UPDATE: fp32 state M_l (in/out); FFG: state out; PLAIN: C
    void* mop;            // UPDATE: operand-type copy of M_l (nullable for fp32)
    const float* eself;   // UPDATE: X_l from the error phase (nullable for the top layer)
    float prec;           // ERROR: P_{l-1}
    int slot_base;        // ERROR: first energy partial slot of this problem
    int ksplit;           // K ranges per tile (<= 1: none); the last range to finish runs the epilogue
    int ksplit_pad;
    float* part;          // split-K: fp32 partial tiles [tiles_m * tiles_n * ksplit x BM * BN]
    int* count;           // split-K: finished ranges per tile [tiles_m * tiles_n], zero between launches
};

// Most K ranges a split-K tile is cut into.
constexpr int kMaxSplit = 8;

// Problems of one grouped launch, passed by value in the kernel arguments.
constexpr int kMaxProblems = 16;
struct ProblemSet {
    Problem p[kMaxProblems];
    int n;
};

static_assert(sizeof(Problem) % 8 == 0, "Problem is copied as 64-bit words");
struct ProblemWords { uint64_t w[sizeof(Problem) / 8]; };

// Copy one problem out of the kernarg segment (address space 4) word by word.
__device__ __forceinline__ Problem load_problem(const __attribute__((address_space(4))) Problem* src) {
    typedef const __attribute__((address_space(4))) uint64_t KWord;
    KWord* w = (KWord*)src;
    ProblemWords pw;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(Problem) / 8); ++i) pw.w[i] = w[i];
    return __builtin_bit_cast(Problem, pw);
}

struct PhaseArgs {
    int act;
    float eta, act_reg;
    float alpha, beta;          // PLAIN
    float* energy_part;         // [nslots x ldp] per-row partial energies (nullable)
    int ldp, nslots;
    float* energy_out;          // UPDATE prologue: row energies of step t (nullable)
    int batch, t;
    const int* row_req;         // ragged: request of each row (nullable)
    const int* done_at;         // ragged: first step a request no longer runs
    int tile_order;             // TILE_INTERLEAVED or TILE_CONTIGUOUS (see phase_grid)
    int k_stagger;              // > 1: K sweeps of tile (tm, tn) start (tm + tn) % k_stagger stages in
    const int* act_tm;          // ragged: row tiles with a row still running, increasing (nullable)
    const int* act_count;       // ragged: their number
    int nt_store;               // settling epilogues store their full rows non-temporally
    int nt_load;                // settling epilogues load their fp32 state rows non-temporally
};

// How a phase's tiles are dealt over the XCDs.
enum TileOrder { TILE_INTERLEAVED = 0, TILE_CONTIGUOUS = 1 };

// ------------------------------------------------------------ scalar helpers

// tanh(x) = sign(x) (1 - 2 / (exp(2|x|) + 1)), from the definition, with the
// hardware exp2 and reciprocal.  Absolute error ~1e-7 (relative error grows
// only where |tanh| is below ~1e-3, where the absolute error is what the
// relaxation sees); saturates to +-1 for large |x|.
__device__ __forceinline__ float fast_tanh(float x) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(fabsf(x) * 2.8853900817779268f);  // exp(2|x|)
    const float t = __builtin_fmaf(-2.f, __builtin_amdgcn_rcpf(e + 1.f), 1.f);
    return copysignf(t, x);
}

// f(pre) and f'(pre) together (Activation.cs:34-132; GELU-tanh and its
// derivative from pre, Layers.cs:42-50 and Autograd.cs:313-318), sharing the
// one transcendental evaluation both need.  Multiply-adds are written out
// (fmaf) and nothing else is contracted, here or in fast_tanh, so f(pre) has
// the same bits in every epilogue whether or not f'(pre) is used beside it:
// the FFG warm start's M_{l-1} = f(W_l M_l + b) and the first error phase's f
// of the same pre-activation must agree exactly (their difference is the
// error, exactly zero in the reference).
__device__ __forceinline__ void act_eval(int act, float x, float& y, float& dy) {
#pragma clang fp contract(off)
    switch (act) {
    case ACT_TANH: {
        y = fast_tanh(x);
        dy = __builtin_fmaf(-y, y, 1.f);
        break;
    }
    case ACT_RELU:
        y = x > 0.f ? x : 0.f;
        dy = x > 0.f ? 1.f : 0.f;
        break;
    case ACT_SIGMOID: {
        y = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
        dy = __builtin_fmaf(-y, y, y);
        break;
    }
    case ACT_GELU: {
        // 0.5 x (1 + tanh(u)) with u = c (x + a x^3) is x s, s = 1 / (1 + exp(-2u))
        // (the identity (1 + tanh(u)) / 2 = sigmoid(2u)); its derivative is
        // s + x s (1 - s) 2 c (1 + 3 a x^2).  One exp2 and one reciprocal, as
        // fast_tanh takes, and six fewer VALU operations than going through it.
        // Saturates to x (dy 1) for large x and to -0 (dy 0) for very negative x.
        const float c = 0.7978845608f, a = 0.044715f;
        const float x2 = x * x;
        const float v = __builtin_fmaf(a * x2, x, x);                                   // x + a x^3
        const float e = __builtin_amdgcn_exp2f(v * (-2.f * c * 1.4426950408889634f));   // exp(-2u)
        const float s = __builtin_amdgcn_rcpf(1.f + e);
        y = x * s;
        const float k = __builtin_fmaf(6.f * a * c, x2, 2.f * c);                      // du/dx times 2
        dy = __builtin_fmaf(y * (1.f - s), k, s);
        break;
    }
    default:
        y = x;
        dy = 1.f;
    }
}

__device__ __forceinline__ float act_f(int act, float x) {
    float y, dy;
    act_eval(act, x, y, dy);
    return y;
}

// Round-to-nearest-even fp32 -> bf16 with NaN kept NaN (TensorUtils.cs:386-395).
__device__ __forceinline__ uint16_t to_bf16(float x) {
    __bf16 h = (__bf16)x;  // v_cvt_pk_bf16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ uint16_t to_f16(float x) {
    _Float16 h = (_Float16)x;  // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// store4 writes elements idx .. idx+3 (idx a multiple of 4) in one access;
// the conversions round to nearest even, as the one-element stores do.
template <typename OP> struct OpTraits;
template <> struct OpTraits<float> {
    static constexpr int bytes = 4;
    __device__ static void store(void* base, size_t idx, float v) { gst((float*)base + idx, v); }
    __device__ static void store4(void* base, size_t idx, f32x4 v) { gst4((float*)base + idx, v); }
    __device__ static float load(const void* base, size_t idx) { return ((const float*)base)[idx]; }
};
template <> struct OpTraits<bf16_t> {
    static constexpr int bytes = 2;
    __device__ static void store(void* base, size_t idx, float v) { gst((uint16_t*)base + idx, to_bf16(v)); }
    __device__ static u32x2 pack4(f32x4 v) { return __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf16x4)); }
    __device__ static void store4(void* base, size_t idx, f32x4 v) { gst4((uint16_t*)base + idx, pack4(v)); }
    __device__ static float load(const void* base, size_t idx) {
        return __uint_as_float((uint32_t)((const uint16_t*)base)[idx] << 16);
    }
};
template <> struct OpTraits<f16_t> {
    static constexpr int bytes = 2;
    __device__ static void store(void* base, size_t idx, float v) { gst((uint16_t*)base + idx, to_f16(v)); }
    __device__ static u32x2 pack4(f32x4 v) { return __builtin_bit_cast(u32x2, __builtin_convertvector(v, f16x4)); }
    __device__ static void store4(void* base, size_t idx, f32x4 v) { gst4((uint16_t*)base + idx, pack4(v)); }
    __device__ static float load(const void* base, size_t idx) {
        return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)base)[idx]);
    }
};

// One 32-byte K chunk of a 32x32 block with 16-bit operands: a and b hold
// this lane's 16 bytes (fp32 operands are issued per K component in the main
// loop itself).
template <typename OP> __device__ __forceinline__ void mfma_chunk(f32x16& acc, const u32x4& a, const u32x4& b);
template <> __device__ __forceinline__ void mfma_chunk<bf16_t>(f32x16& acc, const u32x4& a, const u32x4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
template <> __device__ __forceinline__ void mfma_chunk<f16_t>(f32x16& acc, const u32x4& a, const u32x4& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

// Workgroup ids are dealt round-robin over the XCDs (each with its own L2):
// XCD x runs blocks x, x + 8, x + 16, ...
constexpr int kXcds = 8;

// Share of a problem's n tiles that XCD x runs: [lo, lo + cnt).  The shares
// of the 8 XCDs tile [0, n) exactly and differ in size by at most one.
__host__ __device__ __forceinline__ void xcd_share(int n, int x, int& lo, int& cnt) {
    lo = n * x / kXcds;
    cnt = n * (x + 1) / kXcds - lo;
}

// Sum of a row's energy partials over the slots, in slot order.  The loads
// go out eight at a time ahead of the adds (one dependent load per slot would
// pay the memory latency nslots times).
__device__ __forceinline__ float sum_slots(const float* part, int ldp, int nslots, int row) {
    float s = 0.f;
    int k = 0;
    for (; k + 8 <= nslots; k += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gld(part + (size_t)(k + j) * ldp + row);
#pragma unroll
        for (int j = 0; j < 8; ++j) s += v[j];
    }
    for (; k < nslots; ++k) s += gld(part + (size_t)k * ldp + row);
    return s;
}

// Row activity of the ragged path: the row's request still runs at step t.
__device__ __forceinline__ bool row_active(const PhaseArgs& a, int row) {
    return a.row_req == nullptr || a.t < gld(a.done_at + gld(a.row_req + row));
}

// LDS layout of one pipeline stage: rows of RB bytes (the K slice of one A or
// B row), A rows first, then B rows.  The 16-byte units of row R are stored
// permuted, unit u at u ^ ((R / (256 / RB)) % (RB / 16)): consecutive rows
// then cover all 64 four-byte banks (256 bytes) before a bank repeats, so the
// fragment reads (32 consecutive rows x 2 units per wave, one ds_read_b128
// each) are conflict-free.  For 64-byte rows this was measured on gfx950 with
// SQ_LDS_BANK_CONFLICT (zero); XOR keys built from other row bits leave a
// 2-way conflict.
template <int RB> __device__ __forceinline__ int swz(int row, int unit) {
    return unit ^ ((row / (256 / RB)) % (RB / 16));
}
// Row-major B stages (EPI_PLAIN_KN): 16-byte unit u of K row k sits at unit
// u ^ kn_swz(k).  A transposing fragment read of 32 lanes covers four K rows
// and the same 64 bytes of each; the XOR puts those four pieces on four
// different 64-byte bank windows (LDS: 64 banks of 4 bytes).  Rows of 256 or
// more bytes are a whole number of bank periods, so rows k % 4 = 0..3 take
// windows 0..3 by the XOR alone; 128-byte rows (BN = 64) already alternate
// halves, and the XOR separates k and k + 2.
template <int BN> __device__ __forceinline__ int kn_swz(int k) {
    return BN >= 128 ? (k & 3) * 4 : ((k >> 1) & 1) * 4;
}
// One 32 x 32 x 16 MFMA operand fragment from a stage region that holds K
// rows of W 16-bit elements (a row-major B, or a transposed A), laid out by
// kn_swz<W>: lane l takes element x0 + l % 32 of K rows 16c + 8 (l / 32) +
// 0..7, in two transposing reads of four rows each.  In each group of 16
// lanes, lane i reads row kbase + i / 4 at elements 4 (i % 4) .. + 3 of the
// group's 16, and lane j receives element j % 4 of lanes j / 4, 4 + j / 4,
// 8 + j / 4 and 12 + j / 4, i.e. element j of rows kbase .. kbase + 3.
template <int W> __device__ __forceinline__ u32x4 tr_fragment(const char* region, int c, int x0) {
    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int x = x0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    u32x2 h[2];
    static_for<0, 2>([&](auto Hc) PCD_INLINE {
        const int k = 16 * c + 8 * half + 4 * decltype(Hc)::value + ((lane & 15) >> 2);
        const char* p = region + k * (W * 2) + ((x * 2) ^ (kn_swz<W>(k) * 16));
        h[decltype(Hc)::value] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                       (__attribute__((address_space(3))) v4i16*)(__attribute__((address_space(3))) char*)p));
    });
    return u32x4{h[0][0], h[0][1], h[1][0], h[1][1]};
}

// Build-time tile parameters (K bytes per row per stage: *_RB; LDS ring
// stages: *_NS; workgroups per CU the registers are sized for: OCC).  The
// defaults are the fastest measured on MI355X for the settling phases and the
// GEMM provider; a -D on the compiler line overrides one to measure another.
#ifndef PCD_ERR_PD
#define PCD_ERR_PD 3   // error epilogue: blocks whose M operands are in flight
#endif
#ifndef PCD_EPI_BATCH
#define PCD_EPI_BATCH 1   // epilogue operand loads in batches of PD blocks (0: one block at a time)
#endif
#ifndef PCD_BIG_RB
#define PCD_BIG_RB 128
#endif
#ifndef PCD_BIG_NS
#define PCD_BIG_NS 2
#endif
#ifndef PCD_MID_RB
#define PCD_MID_RB 64
#endif
#ifndef PCD_MID_NS
#define PCD_MID_NS 4
#endif
#ifndef PCD_OCC_SMALL
#define PCD_OCC_SMALL 2
#endif
#ifndef PCD_SMALL_NS
#define PCD_SMALL_NS 4
#endif
#ifndef PCD_SMALL_RB
#define PCD_SMALL_RB 64
#endif
#ifndef PCD_SMALL_RB16
#define PCD_SMALL_RB16 128
#endif
#ifndef PCD_KSW_NS
#define PCD_KSW_NS 3   // the K-shared 32 x 32 tile: 48 KB ring, three workgroups per CU
#endif
#ifndef PCD_KSW_OCC
#define PCD_KSW_OCC 3
#endif
#ifndef PCD_WD_NS
#define PCD_WD_NS 3    // direct-weight tile: 24 KB ring, two stages of lead (3, 4, 5 and 6 measured within 1%)
#endif
#ifndef PCD_WD_OCC
#define PCD_WD_OCC 3
#endif
template <int BM, int BN, int OPB = 4, bool WDIR = false> struct TileCfg {
    // 256 x 256 runs 8 waves (2 x 4 of 128 x 64: two waves per SIMD share the
    // MFMA pipe) over 128-byte K stages, double buffered (128 KB of LDS, one
    // workgroup per CU).  The other tiles run 4 waves (2 x 2) with rings of at
    // most 80 KB, so two workgroups fit a CU.  Their stages are 64 bytes per
    // row, except 64-row tiles on 16-bit operands: 128 bytes, one whole cache
    // line of every weight row per stage, which is what streams best from HBM
    // when the batch is small (the weights dominate the traffic).
    static constexpr bool BIG = BM == 256 && BN == 256;
    // 32 x 32 is one output block whose K the 4 waves share: each stage holds
    // 64 K elements per row (256 bytes of fp32, 128 of 16-bit operands) and
    // wave w takes the w-th quarter of every stage, so a tile's K sweep takes
    // a quarter of the MFMA issue time of a 64 x 64 tile's.  The waves' sums
    // meet in LDS after the loop.
    static constexpr bool KSW = BM == 32 && BN == 32;
    static constexpr bool WD = WDIR;
    // WD (direct weights, 64 x 128 on 16-bit operands only): the weight
    // operand is read from a fragment-major copy straight into registers
    // (each wave's 1 KB fragment of a 16-deep K chunk is one contiguous,
    // non-temporal 16-byte-per-lane load) and only the batch rows go through
    // LDS.  Each of the 4 waves owns all 64 rows and 32 columns, so no two
    // waves read the same weights.  The small-batch settlings, which stream
    // every weight once per phase, are bound by that stream.
    static_assert(!WDIR || (BM == 64 && BN == 128 && OPB == 2), "direct weights: 64 x 128 tiles of 16-bit operands");
    static constexpr int KW = KSW ? 4 : 1;                 // waves sharing one block's K
    static constexpr int WM = (KSW || WD) ? 1 : 2, WN = (BIG || WD) ? 4 : KSW ? 1 : 2;
    static constexpr int NWAVES = WM * WN * KW, NT = 64 * NWAVES;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr bool MID = BM == 128 && BN == 128;
    static constexpr int RB = BIG ? PCD_BIG_RB : MID ? PCD_MID_RB : KSW ? 64 * OPB : (BM == 64 && OPB == 2) ? PCD_SMALL_RB16 : PCD_SMALL_RB;   // K bytes per row per stage
    static constexpr int UNITS = RB / 16;                  // 16-byte units per row
    static constexpr int NC = RB / 32;                     // 32-byte MFMA chunks per stage
    static constexpr int NCW = NC / KW;                    // chunks of a stage one wave takes
    static constexpr int LDS_ROWS = WD ? BM : BM + BN;     // operand rows a stage holds in LDS
    static constexpr int stage_bytes = LDS_ROWS * RB;
    static constexpr int NS_WANT = WD ? PCD_WD_NS : BIG ? PCD_BIG_NS : MID ? PCD_MID_NS : KSW ? PCD_KSW_NS : (BM + BN >= 320) ? 3 : PCD_SMALL_NS;
    static constexpr int NS = (BIG || WD) ? NS_WANT : (NS_WANT * stage_bytes <= 80 * 1024 ? NS_WANT : 80 * 1024 / stage_bytes);   // stages in the LDS ring
    static constexpr int D = NS - 1;                       // prefetch distance (stages)
    static constexpr int OCC = BIG ? 1 : KSW ? PCD_KSW_OCC : WD ? PCD_WD_OCC : PCD_OCC_SMALL;   // workgroups per CU the registers are sized for
    static constexpr int ROWS_PER_LOAD = 64 * 16 / RB;     // rows one wave-wide 16-byte-per-lane load fills
    static constexpr int QPW = LDS_ROWS / ROWS_PER_LOAD / NWAVES;   // loads per wave per stage
    // vector-memory operations a wave issues per stage (DMA, then weights)
    static constexpr int VPS = QPW + (WD ? NCW : 0);
    static_assert(FM >= 1 && FN >= 1 && QPW >= 1, "tile too small");
    static_assert(LDS_ROWS % (NWAVES * ROWS_PER_LOAD) == 0, "stage rows must split evenly over the waves");
    static_assert(NCW % 2 == 0 || NCW == 1, "fragment buffers alternate within a stage (or per stage)");
    static_assert(D >= 1 && D * VPS < 64, "stage_ready waits on at most 63 loads");
    static_assert(NS * stage_bytes <= 160 * 1024, "LDS ring exceeds the 160 KB of a CU");
    static_assert(64 % (RB / OPB) == 0, "K is padded to 64 elements: a stage's K must divide it");
};

// Energy partial slots one tile column owns (one per wave column).
template <int BM, int BN, bool WD = false> constexpr int energy_slots_per_tile_n() {
    return TileCfg<BM, BN, WD ? 2 : 4, WD>::WN;
}

// Direct global -> LDS copy of 16 bytes per lane (gfx950 global_load_lds_dwordx4):
// lane l's bytes land at LDS address m0 + 16 l.  Issued as inline asm so the
// compiler does not serialise it with a vmcnt(0) before every LDS read; the
// kernel places its own vmcnt waits.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* gaddr, uint32_t lds_addr) {
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gaddr), "s"(lds_addr) : "memory", "m0");
}

// Non-temporal 16-byte load per lane into registers, issued as inline asm so
// that the compiler does not wait for it before the next loads.  The compiler
// does not know the registers are still being written: the kernel waits for
// the load itself (wait_vmcnt_pin) before it reads them, and keeps them
// allocated (pin_regs) until every such load has landed, so no other value
// is placed in them meanwhile.
__device__ __forceinline__ u32x4 gload_nt16(const void* gaddr) {
    u32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(r) : "v"(gaddr) : "memory");
    return r;
}
// s_waitcnt vmcnt(N); the four registers are its operands, so the code that
// reads them stays after it.
template <int N> __device__ __forceinline__ void wait_vmcnt_pin(u32x4 (&w)[4]) {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]) : "n"(N) : "memory");
}
__device__ __forceinline__ void pin_regs(u32x4 (&w)[4]) {
    asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]));
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Row-contiguous stores of one 32 x 32 result block held in the transposed
// layout (lane l: row l % 32, columns 8g + 4(l/32) + k of group g).  Stored as
// it is held, one wave store would write 32 rows x 16 or 32 bytes (32 partial
// cache lines, each its own L2 write); the block goes through an LDS region of
// the wave's own instead (stage_group per group of four columns, then
// flush_block) and leaves as whole 128-byte (fp32) or 64-byte (16-bit) row
// segments.  Rows whose bit is clear in rmask and columns at or past n are not
// written.  LDS accesses of one wave complete in order, so the region needs no
// barrier between its uses.
constexpr int kStageRowBytes = 144;                    // 128 bytes of a row + 16 of padding: conflict-free
constexpr int kStageWaveBytes = 32 * kStageRowBytes;   // one region
template <int BYTES, typename Pack>
__device__ __forceinline__ void stage_group(char* st, int g, f32x4 v, Pack pack) {
    const int lane = threadIdx.x & 63, lr = lane & 31, half = lane >> 5;
    if constexpr (BYTES == 4) *(f32x4*)(st + lr * kStageRowBytes + (8 * g + 4 * half) * 4) = v;
    else *(u32x2*)(st + lr * kStageRowBytes + (8 * g + 4 * half) * 2) = pack(v);
}
// The epilogues' operand loads after block B of NB, PD blocks in flight.
// Loads and stores share vmcnt and may complete out of order with each other,
// so once a block's stores are out, a wait for an older load is a wait for
// every vector-memory operation (the compiler emits vmcnt(0)).  A load issued
// after every block would put the next block's wait behind it: a full memory
// round trip per 32 x 32 block.  The next PD blocks' loads therefore go out
// together after the last block of a batch, and only the batch's first block
// waits (one round trip per PD blocks, its loads all in flight at once).
template <int B, int PD, int NB, typename F> __device__ __forceinline__ void next_operands(F&& load_block) {
#if PCD_EPI_BATCH
    if constexpr ((B + 1) % PD == 0 && B + 1 < NB)
        static_for<B + 1, (B + 1 + PD < NB ? B + 1 + PD : NB)>([&](auto Bc) PCD_INLINE { load_block(Bc); });
#else
    if constexpr (B + PD < NB) load_block(std::integral_constant<int, B + PD>{});
#endif
}

// GNT (compile time): non-temporal global stores.  A runtime choice between a
// non-temporal and a plain store of the same address compiles to one store
// without the hint when both are global, so a runtime `nt` alone stores
// through a generic (flat) pointer, which also counts against the LDS wait
// counter; the 256 x 256 settling epilogues take GNT instead (measured 0.4 to
// 1% faster phases than the flat form).
template <int BYTES, bool GNT = false>
__device__ __forceinline__ void flush_block(const char* st, void* out, size_t ld, int row0, int col0, uint64_t rmask,
                                            int n, bool full, bool nt = false) {
    const int lane = threadIdx.x & 63;
    if constexpr (BYTES == 4) {
        static_for<0, 4>([&](auto Pc) PCD_INLINE {
            const int rr = (lane >> 3) + 8 * decltype(Pc)::value, cc = (lane & 7) * 4;
            const f32x4 w = *(const f32x4*)(st + rr * kStageRowBytes + cc * 4);
            float* dst = (float*)out + (size_t)(row0 + rr) * ld + col0 + cc;
            const bool rv = (rmask >> rr) & 1;
            if (full || (rv && col0 + cc + 3 < n)) {
                if constexpr (GNT) __builtin_nontemporal_store(w, (gf32x4*)dst);
                else if (nt) __builtin_nontemporal_store(w, (f32x4*)dst);
                else gst4(dst, w);
            } else if (rv) {
                static_for<0, 4>([&](auto K) PCD_INLINE {
                    constexpr int k = decltype(K)::value;
                    if (col0 + cc + k < n) gst(dst + k, w[k]);
                });
            }
        });
    } else {
        static_for<0, 2>([&](auto Pc) PCD_INLINE {
            const int rr = (lane >> 2) + 16 * decltype(Pc)::value, cc = (lane & 3) * 8;
            const u32x4 w = *(const u32x4*)(st + rr * kStageRowBytes + cc * 2);
            uint16_t* dst = (uint16_t*)out + (size_t)(row0 + rr) * ld + col0 + cc;
            const bool rv = (rmask >> rr) & 1;
            if (full || (rv && col0 + cc + 7 < n)) {
                if constexpr (GNT) __builtin_nontemporal_store(w, (__attribute__((address_space(1))) u32x4*)dst);
                else if (nt) __builtin_nontemporal_store(w, (u32x4*)dst);
                else *(__attribute__((address_space(1))) u32x4*)dst = w;
            } else if (rv) {
                static_for<0, 8>([&](auto K) PCD_INLINE {
                    constexpr int k = decltype(K)::value;
                    if (col0 + cc + k < n) gst(dst + k, (uint16_t)(w[k / 2] >> (16 * (k % 2))));
                });
            }
        });
    }
}
// The loads' counterpart: an fp32 32 x 32 block read as whole 128-byte rows
// (lane l: row (l/8) + 8p, columns 4(l%8) .. +3 as raw[p]; rows at or past m
// and groups at or past n read as zero), then turned into the transposed
// layout through the wave's region (tr[g] = columns 8g + 4(l/32) .. +3 of row
// l % 32).  Read transposed directly, every four lanes would ask for four
// rows, four times the requests of whole rows.
// GNT: non-temporal global loads (see flush_block).
template <bool GNT = false>
__device__ __forceinline__ void load_block_rows(f32x4 (&raw)[4], const float* src, size_t ld, int row0, int col0,
                                                int m, int n, bool nt = false, bool full = false) {
    const int lane = threadIdx.x & 63;
    static_for<0, 4>([&](auto Pc) PCD_INLINE {
        constexpr int p = decltype(Pc)::value;
        const int rr = (lane >> 3) + 8 * p, cc = (lane & 7) * 4;
        const float* a = src + (size_t)(row0 + rr) * ld + col0 + cc;
        raw[p] = (full || (row0 + rr < m && col0 + cc < n))
                     ? (GNT  ? __builtin_nontemporal_load((const gf32x4*)a)
                        : nt ? __builtin_nontemporal_load((const f32x4*)a)
                             : gld4(a))
                     : f32x4{};
    });
}
__device__ __forceinline__ void transpose_block(char* st, const f32x4 (&raw)[4], f32x4 (&tr)[4]) {
    const int lane = threadIdx.x & 63, lr = lane & 31, half = lane >> 5;
    static_for<0, 4>([&](auto Pc) PCD_INLINE {
        constexpr int p = decltype(Pc)::value;
        *(f32x4*)(st + ((lane >> 3) + 8 * p) * kStageRowBytes + (lane & 7) * 16) = raw[p];
    });
    static_for<0, 4>([&](auto G) PCD_INLINE {
        constexpr int g = decltype(G)::value;
        tr[g] = *(const f32x4*)(st + lr * kStageRowBytes + (8 * g + 4 * half) * 4);
    });
}

template <typename OP> struct PackOp {
    __device__ u32x2 operator()(f32x4 v) const {
        if constexpr (OpTraits<OP>::bytes == 2) return OpTraits<OP>::pack4(v);
        else return u32x2{};
    }
};

typedef const __attribute__((address_space(4))) Problem KProblem;

// The end of a settling phase unit on the K-shared 32 x 32 tile.  On entry
// each of the 4 waves holds its partial sum of the whole block over its
// quarter of K (`acc`, transposed layout: lane l has row l % 32, register
// 4g + k is column 8g + 4(l / 32) + k).  Reduce-scatter through LDS: wave w
// ends with group w (columns 8w + 4(l / 32) .. +3 of its row) summed over the
// waves in wave order; then split-K, if any, per group; then the error or
// update epilogue per group, so each wave evaluates a quarter of the block's
// activations and stores its four columns of each row directly (fp32 states,
// operand-type deltas and state copies).  The error phase's row energies meet
// across the groups through LDS, in group order.  `state` and `bias` are this
// lane's four columns of the epilogue's state operand (M_{l-1} in the error
// phase, X_l or the top layer's M_l in the update phase) and of the bias,
// loaded by the caller before the K sweep.
template <typename OP, int BM, int BN, int EPI>
__device__ __forceinline__ void ksw_settle_tail(const Problem& P, const PhaseArgs& args, const f32x16& acc,
                                                const f32x4 state, const f32x4 bias, char* smem, const int tile,
                                                const int split, const int ks, const int row0, const int col0,
                                                const int tn) {
    using C = TileCfg<BM, BN, OpTraits<OP>::bytes>;
    static_assert(C::KW == 4 && C::FM == 1 && C::FN == 1, "one block shared by four waves");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, half = lane >> 5;
    float* red = (float*)smem;                                   // 4 waves x 16 registers x 64 lanes
    float* ered = (float*)(smem + C::KW * 16 * 64 * 4);          // 4 groups x 32 rows
    __syncthreads();   // every wave is done reading the stage ring
    static_for<0, 16>([&](auto R) PCD_INLINE {
        constexpr int r = decltype(R)::value;
        red[(wave * 16 + r) * 64 + lane] = acc[r];
    });
    __syncthreads();
    f32x4 g;
    static_for<0, 4>([&](auto K) PCD_INLINE {
        constexpr int k = decltype(K)::value;
        float v = red[(4 * wave + k) * 64 + lane];
        static_for<1, C::KW>([&](auto W) PCD_INLINE { v += red[(decltype(W)::value * 16 + 4 * wave + k) * 64 + lane]; });
        g[k] = v;
    });

    if (ks > 1) {
        // Split-K per group, the handshake of the other tiles (see phase_unit):
        // each wave publishes its group's two 64-bit words per lane; the range
        // that finishes last sums every range's group in range order.
        typedef unsigned long long u64;
        gu64* part = (gu64*)(P.part + (size_t)tile * ks * (BM * BN));   // global, not flat: see flush_block
        constexpr int UNIT = BM * BN / 2;
        const int slot = (wave * 64 + lane) * 2;
        auto pack = [](float a, float b) PCD_INLINE { return (u64)__float_as_uint(a) | ((u64)__float_as_uint(b) << 32); };
        __hip_atomic_store(part + (size_t)split * UNIT + slot, pack(g[0], g[1]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part + (size_t)split * UNIT + slot + 1, pack(g[2], g[3]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        wait_vmcnt<0>();
        __syncthreads();
        int* flag = (int*)(ered + C::KW * 32);
        if (tid == 0) *flag = __hip_atomic_fetch_add((gint*)(P.count + tile), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*flag != ks - 1) return;
        if (tid == 0) __hip_atomic_store((gint*)(P.count + tile), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
        u64 pv[kMaxSplit][2];
        static_for<0, kMaxSplit>([&](auto Kc) PCD_INLINE {
            constexpr int k = decltype(Kc)::value;
            if (k < ks && k != split)
                static_for<0, 2>([&](auto Q) PCD_INLINE {
                    pv[k][decltype(Q)::value] = __hip_atomic_load(part + (size_t)k * UNIT + slot + decltype(Q)::value,
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                });
        });
        f32x4 sum{};
        static_for<0, kMaxSplit>([&](auto Kc) PCD_INLINE {
            constexpr int k = decltype(Kc)::value;
            if (k < ks) {
                f32x4 v = g;
                if (k != split)
                    v = f32x4{__uint_as_float((uint32_t)pv[k][0]), __uint_as_float((uint32_t)(pv[k][0] >> 32)),
                              __uint_as_float((uint32_t)pv[k][1]), __uint_as_float((uint32_t)(pv[k][1] >> 32))};
                sum = k == 0 ? v : sum + v;
            }
        });
        g = sum;
    }

    // Row lr of the block, columns col .. col + 3.  The caller read `state` and
    // `bias` whatever the row's state (rows and columns are padded in memory,
    // the padding is zero); only valid rows and columns below N are written.
    const int row = row0 + lr, col = col0 + 8 * wave + 4 * half;
    const bool rok = row < P.M && row_active(args, row);
    const bool cfull = col + 3 < P.N;
    const size_t idx = (size_t)row * P.ldo + col;
    // fp32 (`store4`) and operand-type (`store4_op`) stores of this lane's four
    // columns.
    auto store4 = [&](float* dst, const f32x4& v) PCD_INLINE {
        if (!rok) return;
        if (cfull) {
            gst4(dst + idx, v);
        } else {
            static_for<0, 4>([&](auto K) PCD_INLINE {
                constexpr int k = decltype(K)::value;
                if (col + k < P.N) gst(dst + idx + k, v[k]);
            });
        }
    };
    auto store4_op = [&](void* dst, const f32x4& v) PCD_INLINE {
        if (!rok) return;
        if (cfull) {
            OpTraits<OP>::store4(dst, idx, v);
        } else {
            static_for<0, 4>([&](auto K) PCD_INLINE {
                constexpr int k = decltype(K)::value;
                if (col + k < P.N) OpTraits<OP>::store(dst, idx + k, v[k]);
            });
        }
    };
    if constexpr (EPI == EPI_ERROR) {
        const f32x4 mv = state, bv = bias;   // M_{l-1} and b at (row, col .. col + 3)
        const float P_low = P.prec, inv2p = 0.5f / P.prec, eta = args.eta, lam = args.act_reg;
        f32x4 dv, xv;
        float es = 0.f;
        auto body = [&](auto ActC) PCD_INLINE {
            constexpr int ACT = decltype(ActC)::value;
            static_for<0, 4>([&](auto K) PCD_INLINE {
                constexpr int k = decltype(K)::value;
                float y, dy;
                act_eval(ACT, g[k] + bv[k], y, dy);
                const float m = mv[k];
                const float e = P_low * (m - y);
                dv[k] = dy * e;
                // X = M - eta (e + lambda sign M): the state's own part of its update
                float gr = e;
                if (lam > 0.f) gr += lam * (m > 0.f ? 1.f : (m < 0.f ? -1.f : 0.f));
                xv[k] = m - eta * gr;
                if (rok && col + k < P.N) es += e * e;
            });
        };
        switch (args.act) {
        case ACT_TANH: body(std::integral_constant<int, ACT_TANH>{}); break;
        case ACT_RELU: body(std::integral_constant<int, ACT_RELU>{}); break;
        case ACT_SIGMOID: body(std::integral_constant<int, ACT_SIGMOID>{}); break;
        case ACT_GELU: body(std::integral_constant<int, ACT_GELU>{}); break;
        default: body(std::integral_constant<int, ACT_LINEAR>{}); break;
        }
        if (P.eout) store4(P.eout, xv);
        store4_op(P.dout, dv);
        if (args.energy_part != nullptr) {
            // this group's 8 columns of the row (both half-waves), then the
            // four groups in order
            float v = es * inv2p;
            v += __shfl_xor(v, 32);
            if (half == 0) ered[wave * 32 + lr] = v;
            __syncthreads();
            if (wave == 0 && half == 0 && row < P.M) {
                const float e4 = ((ered[lr] + ered[32 + lr]) + ered[64 + lr]) + ered[96 + lr];
                gst(args.energy_part + (size_t)(P.slot_base + tn * C::WN) * args.ldp + row, e4);
            }
        }
    } else {
        // M_l = X_l + eta G below the top (X_l written by the error phase); the
        // top layer reads M_l itself: M_l -= eta (lambda sign M_l - G).
        const float eta = args.eta, lam = args.act_reg;
        const bool folded = P.eself != nullptr;
        const f32x4 xv = state;   // X_l (or M_l at the top) at (row, col .. col + 3)
        f32x4 mn;
        static_for<0, 4>([&](auto K) PCD_INLINE {
            constexpr int k = decltype(K)::value;
            if (folded) {
                mn[k] = xv[k] + eta * g[k];
            } else {
                float grad = -g[k];
                if (lam > 0.f) grad += lam * (xv[k] > 0.f ? 1.f : (xv[k] < 0.f ? -1.f : 0.f));
                mn[k] = xv[k] - eta * grad;
            }
        });
        store4(P.m, mn);
        if (P.mop) store4_op(P.mop, mn);
    }
}

// LDS of one phase unit: the stage ring, which after the main loop the
// settling epilogues reuse as two store-staging regions per wave and the
// tile's bias.
template <typename OP, int BM, int BN, bool WD = false> constexpr int phase_smem_bytes() {
    using C = TileCfg<BM, BN, OpTraits<OP>::bytes, WD>;
    // The K-shared tile's tail needs its reduce-scatter, the row energies and a
    // flag; the others two store-staging regions per wave and the bias.
    constexpr int STAGE_END = C::KSW ? C::KW * 16 * 64 * 4 + C::KW * 32 * 4 + 16 : 2 * C::NWAVES * kStageWaveBytes + BN * 4;
    return C::NS * C::stage_bytes > STAGE_END ? C::NS * C::stage_bytes : STAGE_END;
}

// One workgroup's share of a phase: virtual block `vblock` of a grid of
// `vgrid` blocks over the `nprob` problems at `kprobs` (constant memory).
// A launch of the phase runs it once per workgroup (vblock = blockIdx.x); a
// persistent launch runs every virtual block of a phase, several per
// workgroup, between grid barriers.  `smem` is the workgroup's LDS of
// phase_smem_bytes() bytes.
template <typename OP, int BM, int BN, int EPI, bool WD = false>
__device__ __forceinline__ void phase_unit(KProblem* kprobs, const int nprob, const PhaseArgs& args, const int vblock,
                                           const int vgrid, char* smem) {
    constexpr int OPB = OpTraits<OP>::bytes;
    using C = TileCfg<BM, BN, OPB, WD>;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // Wave w of a K-shared tile takes chunks [w NCW, (w + 1) NCW) of every
    // stage and the whole block; the other tiles give each wave its own block.
    const int wk = C::KW > 1 ? wave : 0, wmn = C::KW > 1 ? 0 : wave;
    const int wm = wmn / C::WN, wn = wmn % C::WN;
    // Waves that store the tile's results (a K-shared tile's waves all hold the
    // same sums after the reduction; wave 0 stores them).
    const bool writer = C::KW == 1 || wave == 0;

    // Energy of the previous error phase, reduced per row in a fixed order
    // before any tile work (deterministic, no atomics).  The rows go to the
    // last virtual blocks, which run the last problems' tiles (or none): the
    // first problem, the one with the longest K sweep in the small networks
    // whose phases are latency-bound, then starts without this delay.
    if (EPI == EPI_UPDATE && args.energy_out != nullptr) {
        for (int row = (vgrid - 1 - vblock) * C::NT + tid; row < args.batch; row += vgrid * C::NT) {
            gst(args.energy_out + (size_t)args.t * args.batch + row,
                sum_slots(args.energy_part, args.ldp, args.nslots, row));
        }
    }

    // XCD x runs the x-th eighth of every problem's tiles, problem after
    // problem.  Every XCD, and every CU of it (an XCD deals its workgroups
    // round-robin over its CUs), then gets a like share of the long-K and the
    // short-K problems of a phase, and an eighth of one problem is a compact
    // block of tiles that share operand rows in the XCD's L2.
    // TILE_CONTIGUOUS instead gives XCD x one contiguous eighth of the phase's
    // tiles taken in problem order (phases of many tiles per CU, where the
    // balance evens out by itself).
    // A ragged phase with a list of the row tiles still running deals only
    // those: problem q then has n_act x tiles_n x ksplit work units, and row
    // tile index tm below counts along the list.
    const int n_act = args.act_tm != nullptr ? __builtin_amdgcn_readfirstlane(gld(args.act_count)) : -1;
    auto units_of = [&](int q) PCD_INLINE {
        return n_act < 0 ? kprobs[q].tiles : n_act * kprobs[q].tiles_n * max(kprobs[q].ksplit, 1);
    };
    const int x = vblock % kXcds;
    int i = vblock / kXcds, p = 0, local = -1;
    if (args.tile_order == TILE_INTERLEAVED) {
        for (; p < nprob; ++p) {
            int lo, cnt;
            xcd_share(units_of(p), x, lo, cnt);
            if (i < cnt) {
                local = lo + i;
                break;
            }
            i -= cnt;
        }
    } else {
        int total = 0;
        for (int q = 0; q < nprob; ++q) total += units_of(q);
        int lo, cnt;
        xcd_share(total, x, lo, cnt);
        if (i < cnt) {
            int t = lo + i;
            for (; p < nprob; ++p) {
                if (t < units_of(p)) {
                    local = t;
                    break;
                }
                t -= units_of(p);
            }
        }
    }
    if (local < 0) return;  // a spare workgroup of this XCD (the grid is 8 x the largest XCD share)
    const Problem P = load_problem(kprobs + p);
    // Split-K: unit `local` is K range `split` of tile `local / ksplit` (a
    // tile's ranges are consecutive units: mostly on one XCD, but an XCD's
    // share may end inside a tile, so the handshake below does not rely on it).
    const int ks = P.ksplit > 1 ? P.ksplit : 1;
    const int split = local % ks;
    local /= ks;
    // Grouped order: runs of 8 row tiles share one column tile.
    const int G = 8;
    const int rows_m = n_act < 0 ? P.tiles_m : n_act;
    int group = local / (G * P.tiles_n);
    int first_m = group * G;
    int gsize = min(rows_m - first_m, G);
    int in_group = local - group * G * P.tiles_n;
    const int tm_at = first_m + in_group % gsize;
    const int tm = n_act < 0 ? tm_at : __builtin_amdgcn_readfirstlane(gld(args.act_tm + tm_at));
    const int tn = in_group / gsize;
    const int row0 = tm * BM, col0 = tn * BN;

    if (args.row_req != nullptr && n_act < 0) {
        // Any active row in the tile?  The flag borrows the first word of the
        // (not yet used) stage ring, which the full ring leaves no room beside.
        volatile __attribute__((address_space(3))) int* flag = (volatile __attribute__((address_space(3))) int*)smem;
        if (tid == 0) *flag = 0;
        __syncthreads();
        if (tid < BM) {
            const int r = row0 + tid;
            if (r < P.M && row_active(args, r)) *flag = 1;
        }
        __syncthreads();
        const bool any = *flag != 0;
        __syncthreads();
        if (!any) return;
    }

    // The K-shared tile's settling epilogue reads 16 bytes of one state row
    // per lane (and, in the error phase, four biases): loaded here, their
    // latency passes under the K sweep.
    f32x4 epi_state{}, epi_bias{};
    if constexpr (C::KW > 1 && (EPI == EPI_ERROR || EPI == EPI_UPDATE)) {
        const size_t eidx = (size_t)(row0 + (lane & 31)) * P.ldo + col0 + 8 * wave + 4 * (lane >> 5);
        if constexpr (EPI == EPI_ERROR) {
            epi_state = gld4(P.mlow + eidx);
            epi_bias = gld4(P.bias + col0 + 8 * wave + 4 * (lane >> 5));
        } else {
            epi_state = gld4((P.eself != nullptr ? P.eself : P.m) + eidx);
        }
    }

    // ---- main loop
    // fp32 MFMAs take K = 2 each, four per 32-byte chunk: with fewer than four
    // output blocks per wave they rotate over NSPLIT accumulator sets (summed
    // after the loop), so consecutive MFMAs never wait on each other's result.
    constexpr bool F32OP = std::is_same<OP, float>::value;
    constexpr int NSPLIT = (F32OP && C::FM * C::FN < 4) ? 4 / (C::FM * C::FN) : 1;
    f32x16 accs[NSPLIT][C::FM][C::FN];
#pragma unroll
    for (int k = 0; k < NSPLIT; ++k)
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) accs[k][i][j] = f32x16{};

    constexpr int KE = C::RB / OPB;  // K elements per stage
    const int nk_all = P.K / KE;
    const int kb = split * nk_all / ks;             // this unit's stages [kb, kb + nk)
    const int nk = (split + 1) * nk_all / ks - kb;
    // K stagger: tile (tm, tn) sweeps its stages starting at (tm + tn) % S and
    // wrapping round.  The tiles of an XCD that share operand rows then ask for
    // a row's next stage at different times: one takes the L2 miss and the
    // others find the line resident, instead of all of them waiting on the same
    // miss.  The sum over K is taken in that rotated order, so a row's result
    // depends on the row tile it falls in (still the same run to run).
    const int koff = (!C::WD && args.k_stagger > 1 && nk > 0) ? ((tm + tn) % args.k_stagger) % nk : 0;
    // B row-major [K x N] (EPI_PLAIN_KN, _MKKN): ldb is its row pitch, a stage
    // is KE of its rows, and the tile's columns start col0 elements into each
    // row.  A stored [K x M] (EPI_PLAIN_MK, _MKKN) likewise, with lda and row0.
    constexpr bool BKN = EPI == EPI_PLAIN_KN || EPI == EPI_PLAIN_MKKN;
    constexpr bool AKM = EPI == EPI_PLAIN_MK || EPI == EPI_PLAIN_MKKN;
    static_assert(!(AKM || BKN) || (OPB == 2 && C::KW == 1 && !C::WD),
                  "operands read through transposing LDS reads: 16-bit operands, LDS-operand tiles");
    const size_t lda_b = (size_t)P.lda * OPB, ldb_b = (size_t)P.ldb * OPB;
    const char* Ag = AKM ? (const char*)P.A + (size_t)row0 * OPB + (size_t)kb * KE * lda_b
                         : (const char*)P.A + (size_t)row0 * lda_b + (size_t)kb * C::RB;
    const char* Bg = BKN ? (const char*)P.B + (size_t)col0 * OPB + (size_t)kb * KE * ldb_b
                         : (const char*)P.B + (size_t)col0 * ldb_b + (size_t)kb * C::RB;

    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
    const int half = lane >> 5, lr = lane & 31;
    // The settling epilogues (error, update) take each block transposed: the
    // B-side fragment goes in as the MFMA's first operand, so a lane holds one
    // row and runs of four consecutive columns, which those epilogues read and
    // write 16 bytes at a time.
    constexpr bool TRM = EPI == EPI_ERROR || EPI == EPI_UPDATE;
    if constexpr (C::WD) {
        // ---- direct-weight main loop.  Per stage, each wave DMAs its QPW
        // loads of the batch rows into the LDS ring and loads its NCW weight
        // fragments (one per 16-deep K chunk, 1 KB contiguous in the
        // fragment-major copy) into a ring of D register sets.  Stage kt's
        // DMA and weights are issued D stages ahead, DMA first, so waiting
        // until at most (D - 1) * VPS vector-memory operations are in flight
        // retires both; the barrier after the wait publishes every wave's
        // DMA.  Loads past the last stage repeat the last one (in bounds,
        // never read), so every stage issues the same count.  No K stagger:
        // the weight streams of a phase never share rows.
        const size_t kc16 = (size_t)P.K / 16;   // 16-deep K chunks of a weight row
        const char* wsrc = (const char*)P.B + (((size_t)(col0 / 32 + wn) * kc16 + (size_t)kb * C::NCW) * 64 + lane) * 16;
        const char* asrc[C::QPW];
#pragma unroll
        for (int i = 0; i < C::QPW; ++i) {
            const int R = (wave_u * C::QPW + i) * C::ROWS_PER_LOAD + lane / C::UNITS;
            asrc[i] = Ag + (size_t)R * lda_b + swz<C::RB>(R, lane % C::UNITS) * 16;
        }
        auto issue_a = [&](int kt) PCD_INLINE {
            const int kk = min(kt, nk - 1);
            const uint32_t base = lds0 + (kt % C::NS) * C::stage_bytes + wave_u * C::QPW * 1024;
#pragma unroll
            for (int i = 0; i < C::QPW; ++i) lds_dma16(asrc[i] + (size_t)kk * C::RB, base + i * 1024);
        };
        auto issue_w = [&](int kt, u32x4 (&w)[C::NCW]) PCD_INLINE {
            const char* src = wsrc + (size_t)min(kt, nk - 1) * (C::NCW * 1024);
            static_for<0, C::NCW>([&](auto Cc) PCD_INLINE { w[Cc] = gload_nt16(src + decltype(Cc)::value * 1024); });
        };
        static_assert(C::NCW == 4 && C::FN == 1, "the direct-weight ring holds four chunks of one block column");
        u32x4 wr[C::D][C::NCW];
        static_for<0, C::D>([&](auto J) PCD_INLINE {
            issue_a(decltype(J)::value);
            issue_w(decltype(J)::value, wr[decltype(J)::value]);
        });
        // Whole groups of D stages: every stage slot of a group waits, DMAs and
        // refills (the same vector-memory sequence on every path, which the
        // fixed wait counts rely on); slots past the last stage skip only the
        // LDS reads and MFMAs.
        for (int kt0 = 0; kt0 < nk; kt0 += C::D) {
            static_for<0, C::D>([&](auto J) PCD_INLINE {
                constexpr int j = decltype(J)::value;
                const int kt = kt0 + j;
                wait_vmcnt_pin<(C::D - 1) * C::VPS>(wr[j]);
                __syncthreads();
                issue_a(kt + C::D);
                if (kt < nk) {
                    const char* st = smem + (kt % C::NS) * C::stage_bytes;
                    u32x4 fa[C::NCW][C::FM];
                    static_for<0, C::NCW>([&](auto Cc) PCD_INLINE {
                        static_for<0, C::FM>([&](auto I) PCD_INLINE {
                            constexpr int c = decltype(Cc)::value, i = decltype(I)::value;
                            const int R = i * 32 + lr;
                            fa[c][i] = *(const u32x4*)(st + R * C::RB + swz<C::RB>(R, 2 * c + half) * 16);
                        });
                    });
                    static_for<0, C::NCW>([&](auto Cc) PCD_INLINE {
                        static_for<0, C::FM>([&](auto I) PCD_INLINE {
                            constexpr int c = decltype(Cc)::value, i = decltype(I)::value;
                            if constexpr (TRM) mfma_chunk<OP>(accs[0][i][0], wr[j][c], fa[c][i]);
                            else mfma_chunk<OP>(accs[0][i][0], fa[c][i], wr[j][c]);
                        });
                    });
                }
                __builtin_amdgcn_sched_barrier(0);   // the refill follows the MFMAs that read the set
                issue_w(kt + C::D, wr[j]);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        // The last D sets are never read: their loads land before anything
        // else may take their registers.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        static_for<0, C::D>([&](auto J) PCD_INLINE { pin_regs(wr[decltype(J)::value]); });
    } else {
    // This lane's source of each of its wave's QPW loads per stage: combined
    // stage row R = q*ROWS_PER_LOAD + lane/UNITS (A rows, then B rows),
    // physical unit lane%UNITS, which holds logical unit swz(R, lane%UNITS).
    // Row-major B (BKN) instead fills the stage's B region (KE rows of BN
    // elements) as it lies in memory, row after row, each row's 16-byte units
    // permuted by kn_swz so that the transposing fragment reads below are
    // conflict-free: the lane that writes region byte ob copies row ob / (BN
    // OPB), unit (ob % (BN OPB)) / 16 ^ kn_swz(row).  A stage then advances
    // the B source by KE rows.  A transposed A (AKM) fills the A region (KE
    // rows of BM elements) the same way.
    const char* src[C::QPW];
#pragma unroll
    for (int i = 0; i < C::QPW; ++i) {
        const int q = wave_u * C::QPW + i;
        const int R = q * C::ROWS_PER_LOAD + lane / C::UNITS;
        const int unit = swz<C::RB>(R, lane % C::UNITS);
        if (BKN && R >= BM) {
            const int ob = (q * C::ROWS_PER_LOAD - BM) * C::RB + lane * 16;
            const int kr = ob / (BN * OPB);
            src[i] = Bg + (size_t)kr * ldb_b + ((ob % (BN * OPB)) / 16 ^ kn_swz<BN>(kr)) * 16;
        } else if (AKM && R < BM) {
            const int ob = q * C::ROWS_PER_LOAD * C::RB + lane * 16;
            const int kr = ob / (BM * OPB);
            src[i] = Ag + (size_t)kr * lda_b + ((ob % (BM * OPB)) / 16 ^ kn_swz<BM>(kr)) * 16;
        } else {
            src[i] = R < BM ? Ag + (size_t)R * lda_b + unit * 16 : Bg + (size_t)(R - BM) * ldb_b + unit * 16;
        }
    }
    const size_t bstep = BKN ? (size_t)KE * ldb_b : (size_t)C::RB;   // source bytes per stage of B loads
    const size_t astep = AKM ? (size_t)KE * lda_b : (size_t)C::RB;   // ... and of A loads
    auto issue_stage = [&](int kt) PCD_INLINE {
        const uint32_t base = lds0 + (kt % C::NS) * C::stage_bytes + wave_u * C::QPW * 1024;
        int kk = kt + koff;
        if (kk >= nk) kk -= nk;
#pragma unroll
        for (int i = 0; i < C::QPW; ++i) {
            const bool bload = (wave_u * C::QPW + i) * 1024 >= BM * C::RB;   // wave-uniform
            lds_dma16(src[i] + (size_t)kk * (bload ? bstep : astep), base + i * 1024);
        }
    };
    // Fragments of K chunk c (32 bytes per row) of the stage in `slot`.
    auto read_frags = [&](int slot, int c, u32x4* a, u32x4* b) PCD_INLINE {
        const char* st = smem + slot * C::stage_bytes;
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
            if constexpr (AKM) {
                a[i] = tr_fragment<BM>(st, c, wm * C::WTM + i * 32);
            } else {
                const int R = wm * C::WTM + i * 32 + lr;
                a[i] = *(const u32x4*)(st + R * C::RB + swz<C::RB>(R, 2 * c + half) * 16);
            }
        }
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            if constexpr (BKN) {
                b[j] = tr_fragment<BN>(st + BM * C::RB, c, wn * C::WTN + j * 32);
            } else {
                const int R = BM + wn * C::WTN + j * 32 + lr;
                b[j] = *(const u32x4*)(st + R * C::RB + swz<C::RB>(R, 2 * c + half) * 16);
            }
        }
    };
    auto mfmas = [&](const u32x4* a, const u32x4* b) PCD_INLINE {
        if constexpr (F32OP) {
            // K component s of every block before component s + 1 of any.
            static_for<0, 4>([&](auto Sc) PCD_INLINE {
                constexpr int s = decltype(Sc)::value, k = s % NSPLIT;
                static_for<0, C::FM>([&](auto I) PCD_INLINE {
                    static_for<0, C::FN>([&](auto J) PCD_INLINE {
                        constexpr int i = decltype(I)::value, j = decltype(J)::value;
                        const float av = __uint_as_float(a[i][s]), bv = __uint_as_float(b[j][s]);
                        accs[k][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(TRM ? bv : av, TRM ? av : bv,
                                                                            accs[k][i][j], 0, 0, 0);
                    });
                });
            });
        } else {
            static_for<0, C::FM>([&](auto I) PCD_INLINE {
                static_for<0, C::FN>([&](auto J) PCD_INLINE {
                    constexpr int i = decltype(I)::value, j = decltype(J)::value;
                    if constexpr (TRM) mfma_chunk<OP>(accs[0][i][j], b[j], a[i]);
                    else mfma_chunk<OP>(accs[0][i][j], a[i], b[j]);
                });
            });
        }
    };
    // Wait until stage `next` has landed for this wave, given how many later
    // stages are still in flight, then make it visible to all waves.
    auto stage_ready = [&](int next) PCD_INLINE {
        const int later = min(C::D - 1, nk - 1 - next);   // 0 .. D-1
        static_for<0, C::D>([&](auto Kc) PCD_INLINE {
            constexpr int k = decltype(Kc)::value;
            if (later == k) wait_vmcnt<k * C::QPW>();
        });
        __syncthreads();
    };
    constexpr int NC = C::NCW;   // chunks of a stage this wave reads
    u32x4 fa[2][C::FM], fb[2][C::FN];
    // One LDS fragment read after each of the chunk's first MFMAs, the rest of
    // the MFMAs after them.
    constexpr int NMF = C::FM * C::FN * (F32OP ? 4 : 1);   // MFMAs per chunk
    constexpr int NRD = C::FM * (AKM ? 2 : 1) + C::FN * (BKN ? 2 : 1);   // fragment reads per chunk
    auto interleave = [&]() PCD_INLINE {
        // MFMA first: the chunk's first MFMA then waits only on fragments read
        // before it, not on the read just issued (bf16 phases +1%).
        if constexpr (AKM || BKN) {
            constexpr int NP = NMF < NRD ? NMF : NRD;
            static_for<0, NP>([&](auto) PCD_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            });
            if constexpr (NMF > NP) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NP, 0);
            if constexpr (NRD > NP) __builtin_amdgcn_sched_group_barrier(0x100, NRD - NP, 0);
        } else {
            static_for<0, NRD>([&](auto) PCD_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            });
            if constexpr (NMF > NRD) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD, 0);
        }
    };
    const int c0 = wk * C::NCW;   // this wave's first chunk of a stage
    for (int s2 = 0; s2 < C::D && s2 < nk; ++s2) issue_stage(s2);
    stage_ready(0);
    read_frags(0, c0, fa[0], fb[0]);
    // Chunk c's MFMAs run while chunk c+1's fragments are read; the last chunk
    // of a stage runs after the barrier that publishes the next stage, whose
    // first fragments it overlaps.  The last stage is peeled off.
    for (int kt = 0; kt + 1 < nk; ++kt) {
        if (kt + C::D < nk) issue_stage(kt + C::D);
        if constexpr (NC == 1) {
            // One chunk per wave and stage (the K-shared tile on 16-bit
            // operands): its MFMA runs across the barrier, and the next
            // stage's fragments are read into the same registers after it.
            mfmas(fa[0], fb[0]);
            stage_ready(kt + 1);
            read_frags((kt + 1) % C::NS, c0, fa[0], fb[0]);
        } else {
            static_for<0, NC>([&](auto Cc) PCD_INLINE {
                constexpr int c = decltype(Cc)::value;
                if constexpr (c + 1 < NC) {
                    read_frags(kt % C::NS, c0 + c + 1, fa[(c + 1) & 1], fb[(c + 1) & 1]);
                } else {
                    stage_ready(kt + 1);
                    read_frags((kt + 1) % C::NS, c0, fa[0], fb[0]);
                }
                mfmas(fa[c & 1], fb[c & 1]);
                interleave();
            });
        }
    }
    static_for<0, NC>([&](auto Cc) PCD_INLINE {
        constexpr int c = decltype(Cc)::value;
        if constexpr (c + 1 < NC) read_frags((nk - 1) % C::NS, c0 + c + 1, fa[(c + 1) & 1], fb[(c + 1) & 1]);
        mfmas(fa[c & 1], fb[c & 1]);
    });
    }   // LDS-operand main loop
    static_for<1, NSPLIT>([&](auto Kc) PCD_INLINE {
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) accs[0][i][j] += accs[decltype(Kc)::value][i][j];
    });
    f32x16 (&acc)[C::FM][C::FN] = accs[0];
    // The settling epilogues take each block transposed (TR): the B-side
    // fragment went in as the MFMA's first operand, so a lane holds one row
    // and runs of four consecutive columns (the result layout at the top of
    // this file with rows and columns exchanged).
    constexpr bool TR = EPI == EPI_ERROR || EPI == EPI_UPDATE;
    if constexpr (C::KW > 1 && TR) {
        ksw_settle_tail<OP, BM, BN, EPI>(P, args, acc[0][0], epi_state, epi_bias, smem, local, split, ks, row0, col0,
                                         tn);
        return;
    }
    if constexpr (C::KW > 1) {
        // The waves' partial sums of the block meet in LDS (lane-contiguous,
        // conflict-free); every wave adds them in wave order, so all of them
        // hold the same block.
        float* red = (float*)smem;
        __syncthreads();   // every wave is done reading the stage ring
        static_for<0, 16>([&](auto R) PCD_INLINE {
            constexpr int r = decltype(R)::value;
            red[(wave * 16 + r) * 64 + lane] = acc[0][0][r];
        });
        __syncthreads();
        static_for<0, 16>([&](auto R) PCD_INLINE {
            constexpr int r = decltype(R)::value;
            float v = red[r * 64 + lane];
            static_for<1, C::KW>([&](auto W) PCD_INLINE { v += red[(decltype(W)::value * 16 + r) * 64 + lane]; });
            acc[0][0][r] = v;
        });
    }

    // ---- split-K: publish this range's partial tile; the range that finishes
    // last sums all of them in range order (the same sum whichever finishes
    // last) and goes on to the epilogue, the others are done.
    // The partials move with device-scope (agent) atomic stores and loads,
    // which gfx950 performs at the device's coherence point (sc1: no XCD's L2
    // keeps them non-coherently), so ranges on different XCDs see each
    // other's partials.  Ordering: every thread of a range waits until its
    // partial stores are acknowledged (vmcnt(0)) before the workgroup barrier,
    // and only then does thread 0 bump the tile's counter (a device-scope
    // atomic); the range that reads ks - 1 issues its loads of the others'
    // partials only after its bump has returned (the flag in LDS and the
    // barrier).  Every store a counter bump follows has therefore completed
    // at the coherence point before the last range's loads are issued.
    // A release-acquire bump states the same in the language's memory model,
    // but gfx950 implements it with an L2 write-back and an L2 invalidate per
    // range (buffer_wbl2 / buffer_inv), which also discards the other
    // workgroups' cached operands: measured +10% on a split update phase
    // (1024-wide fp32 network), -5% on a whole classification settling.
    if (ks > 1) {
        const int tile = local;
        // Lane-contiguous layout: block (i, j) of this wave holds each lane's 16
        // accumulators as 8 consecutive 64-bit pairs (a wave's block is 4 KB).
        typedef unsigned long long u64;
        gu64* part = (gu64*)(P.part + (size_t)tile * ks * (BM * BN));   // global, not flat: see flush_block
        auto slot_of = [&](int i, int j) PCD_INLINE { return (((wmn * C::FM + i) * C::FN + j) * 64 + lane) * 8; };
        constexpr int UNIT = BM * BN / 2;   // 64-bit words of one partial tile
        gu64* mine = part + (size_t)split * UNIT;
        if (writer) {
            static_for<0, C::FM>([&](auto I) PCD_INLINE {
                static_for<0, C::FN>([&](auto J) PCD_INLINE {
                    constexpr int i = decltype(I)::value, j = decltype(J)::value;
                    static_for<0, 8>([&](auto Q) PCD_INLINE {
                        constexpr int q = decltype(Q)::value;
                        const u64 w =
                            (u64)__float_as_uint(acc[i][j][2 * q]) | ((u64)__float_as_uint(acc[i][j][2 * q + 1]) << 32);
                        __hip_atomic_store(mine + slot_of(i, j) + q, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    });
                });
            });
        }
        wait_vmcnt<0>();      // this lane's partial stores are complete
        __syncthreads();      // ... every lane's; the stage ring is no longer read
        int* flag = (int*)smem;
        if (tid == 0)
            *flag = __hip_atomic_fetch_add((gint*)(P.count + tile), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const bool last = *flag == ks - 1;
        if (!last) return;
        if (tid == 0) __hip_atomic_store((gint*)(P.count + tile), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
        // Per block, four ranges at a time: their words are all requested
        // before any is summed (two round trips for eight ranges), and the sum
        // runs over the ranges in order.
        constexpr int KG = 4;
        static_for<0, C::FM>([&](auto I) PCD_INLINE {
            static_for<0, C::FN>([&](auto J) PCD_INLINE {
                constexpr int i = decltype(I)::value, j = decltype(J)::value;
                float lo[8], hi[8];
                static_for<0, kMaxSplit / KG>([&](auto Gc) PCD_INLINE {
                    constexpr int g = decltype(Gc)::value;
                    if (g * KG < ks) {
                        u64 pv[KG][8];
                        static_for<0, KG>([&](auto K) PCD_INLINE {
                            constexpr int k = g * KG + decltype(K)::value;
                            if (k < ks && k != split)
                                static_for<0, 8>([&](auto Q) PCD_INLINE {
                                    pv[decltype(K)::value][decltype(Q)::value] =
                                        __hip_atomic_load(part + (size_t)k * UNIT + slot_of(i, j) + decltype(Q)::value,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                });
                        });
                        static_for<0, 8>([&](auto Q) PCD_INLINE {
                            constexpr int q = decltype(Q)::value;
                            static_for<0, KG>([&](auto K) PCD_INLINE {
                                constexpr int k = g * KG + decltype(K)::value;
                                if (k < ks) {
                                    float a, b;
                                    if (k == split) {
                                        a = acc[i][j][2 * q];
                                        b = acc[i][j][2 * q + 1];
                                    } else {
                                        a = __uint_as_float((uint32_t)pv[decltype(K)::value][q]);
                                        b = __uint_as_float((uint32_t)(pv[decltype(K)::value][q] >> 32));
                                    }
                                    lo[q] = k == 0 ? a : lo[q] + a;
                                    hi[q] = k == 0 ? b : hi[q] + b;
                                }
                            });
                        });
                    }
                });
                static_for<0, 8>([&](auto Q) PCD_INLINE {
                    acc[i][j][2 * decltype(Q)::value] = lo[decltype(Q)::value];
                    acc[i][j][2 * decltype(Q)::value + 1] = hi[decltype(Q)::value];
                });
            });
        });
    }

    // ---- epilogue
    // FFG and plain epilogues (result layout as at the top of this file): row
    // of register r of a block in row-block i: 8*(r/4) + 4*half + r%4.
    auto row_of = [&](int i, int r) PCD_INLINE { return row0 + wm * C::WTM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3); };
    auto col_of = [&](int j) PCD_INLINE { return col0 + wn * C::WTN + j * 32 + lr; };
    // In the plain epilogue a full tile (every row and column valid, no ragged
    // rows) takes a path with no per-element test: each element's offset is the
    // block's base plus a per-register row step.  Partial tiles test every
    // element.
    const int ldo = P.ldo;
    auto rstep = [&](int r) PCD_INLINE { return (size_t)(8 * (r >> 2) + (r & 3)) * ldo; };
    auto base_of = [&](int i, int j) PCD_INLINE { return (size_t)row_of(i, 0) * ldo + col_of(j); };
    const bool full = row0 + BM <= P.M && col0 + BN <= P.N && args.row_req == nullptr;
    // The settling epilogues (TR): lane l holds row l % 32 of each block, and
    // register 4g + k of block (i, j) is column tcol(j, g) + k.  Every group of
    // four registers is loaded in one 16-byte access, the row and column tests
    // are made per lane and group, not per element, and results leave through
    // the wave's LDS region as whole row segments (store_block).  Columns at or
    // past N are never written (the padding of the states stays zero).
    auto trow = [&](int i) PCD_INLINE { return row0 + wm * C::WTM + i * 32 + lr; };
    auto tcol = [&](int j, int g) PCD_INLINE { return col0 + wn * C::WTN + j * 32 + 8 * g + 4 * half; };
    char* wstage = smem + 2 * wave_u * kStageWaveBytes;   // X / M_l values
    const bool ntst = args.nt_store != 0, ntld = args.nt_load != 0;
    char* wstage2 = wstage + kStageWaveBytes;             // D / operand-copy values
    if constexpr (TR) __syncthreads();   // every wave is done reading the stage ring
    if constexpr (EPI == EPI_ERROR) {
        // On the 256 x 256 tile (the large 16-bit models), one copy of the
        // epilogue per activation, chosen once per tile: the per-element
        // activation switch would otherwise stay in the code (measured 15%
        // of the epilogue).  Smaller tiles keep one generic copy, which
        // compiles several times faster.
        auto epilogue = [&](auto ActC, auto GntC) PCD_INLINE {
            constexpr int ACT = decltype(ActC)::value;
            constexpr bool GNT = decltype(GntC)::value;   // non-temporal global loads and stores
            // Blocks b = i*FN + j in order, their M_{l-1} operands loaded PD
            // blocks at a time (next_operands).
            constexpr int NB = C::FM * C::FN, PD = NB < PCD_ERR_PD ? NB : PCD_ERR_PD;
            const float P_low = P.prec, inv2p = 0.5f / P.prec;
            const float eta = args.eta, lam = args.act_reg;
            const bool want_energy = args.energy_part != nullptr;
            // The tile's bias, once into LDS (registers are short on the
            // 256 x 256 tile); each group reads its four values from there.
            float* sbias = (float*)(smem + 2 * C::NWAVES * kStageWaveBytes);
            for (int c = tid * 4; c < BN; c += C::NT * 4)
                *(f32x4*)(sbias + c) = col0 + c < P.N ? gld4(P.bias + col0 + c) : f32x4{};
            __syncthreads();
            f32x4 mraw[PD][4];
            auto load_block = [&](auto Bc) PCD_INLINE {
                constexpr int b = decltype(Bc)::value, i = b / C::FN, j = b % C::FN;
                load_block_rows<GNT>(mraw[b % PD], P.mlow, ldo, row0 + wm * C::WTM + i * 32, col0 + wn * C::WTN + j * 32,
                                P.M, P.N, ntld);
            };
            static_for<0, PD>([&](auto Bc) PCD_INLINE { load_block(Bc); });
            float esum = 0.f;
            bool rok = false;
            uint64_t rmask = 0;
            static_for<0, NB>([&](auto Bc) PCD_INLINE {
                constexpr int b = decltype(Bc)::value, i = b / C::FN, j = b % C::FN;
                const int row = trow(i);
                if constexpr (j == 0) {
                    esum = 0.f;
                    rok = row < P.M && row_active(args, row);
                    rmask = __ballot(rok);
                }
                f32x4 mv[4];
                transpose_block(wstage, mraw[b % PD], mv);
                static_for<0, 4>([&](auto G) PCD_INLINE {
                    constexpr int g = decltype(G)::value;
                    const int col = tcol(j, g);
                    const f32x4 bv = *(const f32x4*)(sbias + (col - col0));
                    f32x4 dv, xv, ev;
                    static_for<0, 4>([&](auto K) PCD_INLINE {
                        constexpr int k = decltype(K)::value;
                        const float pre = acc[i][j][4 * g + k] + bv[k];
                        float y, dy;
                        act_eval(ACT >= 0 ? ACT : args.act, pre, y, dy);
                        const float e = P_low * (mv[g][k] - y);
                        dv[k] = dy * e;
                        ev[k] = e;
                    });
                    // The state's own part of its update, folded here while
                    // M_{l-1} is in registers: X = M - eta (e + lambda sign M).
                    // The update phase then only adds eta * (W^T D).  lambda = 0
                    // (no activity regularisation) takes a branch of its own, with
                    // the same bits (e + 0 is e): as one expression the sign's
                    // compares and selects ran for every element whatever lambda.
                    if (lam > 0.f) {
                        static_for<0, 4>([&](auto K) PCD_INLINE {
                            constexpr int k = decltype(K)::value;
                            const float m = mv[g][k];
                            const float gr = ev[k] + lam * (m > 0.f ? 1.f : (m < 0.f ? -1.f : 0.f));
                            xv[k] = m - eta * gr;
                        });
                    } else {
                        static_for<0, 4>([&](auto K) PCD_INLINE {
                            constexpr int k = decltype(K)::value;
                            xv[k] = mv[g][k] - eta * ev[k];
                        });
                    }
                    if (want_energy) {   // the row energies only when a caller reads them
                        float es = 0.f;
                        if (rok && col + 3 < P.N) {
                            es = ev[0] * ev[0] + ev[1] * ev[1] + ev[2] * ev[2] + ev[3] * ev[3];
                        } else if (rok) {
                            static_for<0, 4>([&](auto K) PCD_INLINE {
                                constexpr int k = decltype(K)::value;
                                if (col + k < P.N) es += ev[k] * ev[k];
                            });
                        }
                        esum += es * inv2p;
                    }
                    stage_group<4>(wstage, g, xv, PackOp<OP>{});
                    stage_group<OPB>(wstage2, g, dv, PackOp<OP>{});
                });
                const int brow = row0 + wm * C::WTM + i * 32, bcol = col0 + wn * C::WTN + j * 32;
                if (P.eout && writer) flush_block<4, GNT>(wstage, P.eout, ldo, brow, bcol, rmask, P.N, full, ntst);
                if (writer) flush_block<OPB, GNT>(wstage2, P.dout, ldo, brow, bcol, rmask, P.N, full, ntst);
                next_operands<b, PD, NB>(load_block);
                if constexpr (j == C::FN - 1) {
                    if (want_energy) {
                        // The two half-waves hold the two column halves of each group.
                        const float v = esum + __shfl_xor(esum, 32);
                        if (half == 0 && row < P.M && writer) {
                            const int slot = P.slot_base + tn * C::WN + wn;
                            gst(args.energy_part + (size_t)slot * args.ldp + row, v);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);  // the next block starts after this one's loads are issued
            });
        };
        if constexpr (C::BIG) {
            // and per cache policy: non-temporal global accesses when both the
            // loads and the stores are to be non-temporal (the 16-bit default)
            auto per_act = [&](auto ActC) PCD_INLINE {
                if (ntst && ntld) epilogue(ActC, std::true_type{});
                else epilogue(ActC, std::false_type{});
            };
            switch (args.act) {
            case ACT_TANH: per_act(std::integral_constant<int, ACT_TANH>{}); break;
            case ACT_RELU: per_act(std::integral_constant<int, ACT_RELU>{}); break;
            case ACT_SIGMOID: per_act(std::integral_constant<int, ACT_SIGMOID>{}); break;
            case ACT_GELU: per_act(std::integral_constant<int, ACT_GELU>{}); break;
            default: per_act(std::integral_constant<int, ACT_LINEAR>{}); break;
            }
        } else {
            epilogue(std::integral_constant<int, -1>{}, std::false_type{});   // activation chosen per element
        }
    } else if constexpr (EPI == EPI_UPDATE) {
        // M_l = X_l + eta G for the layers below the top, X_l = M_l - eta (E_l +
        // lambda sign M_l) having been written by the error phase; the top
        // layer (E = 0) reads M_l itself: M_l -= eta (lambda sign M_l - G).
        // The operands are loaded PD blocks at a time (next_operands).
        // A whole tile of the 256 x 256 tile (no ragged rows) runs a copy
        // compiled without bounds or row tests (FULL): straight-line loads and
        // stores, no branch around each access, no per-lane row masks
        // (measured: the update epilogue 28 -> 24 us per tile on c5's shapes;
        // the error epilogue, whose arithmetic dominates, gained nothing).
        constexpr int NB = C::FM * C::FN, PD = NB < 3 ? NB : 3;
        const float eta = args.eta, lam = args.act_reg;
        const bool folded = P.eself != nullptr;
        const float* src = folded ? P.eself : P.m;
        auto update = [&](auto FullC, auto GntC) PCD_INLINE {
        constexpr bool FULL = decltype(FullC)::value;
        constexpr bool GNT = decltype(GntC)::value;   // non-temporal global loads and stores
        f32x4 xraw[PD][4];
        auto load_block = [&](auto Bc) PCD_INLINE {
            constexpr int b = decltype(Bc)::value, i = b / C::FN, j = b % C::FN;
            load_block_rows<GNT>(xraw[b % PD], src, ldo, row0 + wm * C::WTM + i * 32, col0 + wn * C::WTN + j * 32,
                                 P.M, P.N, ntld, FULL);
        };
        static_for<0, PD>([&](auto Bc) PCD_INLINE { load_block(Bc); });
        uint64_t rmask = 0;
        static_for<0, NB>([&](auto Bc) PCD_INLINE {
            constexpr int b = decltype(Bc)::value, i = b / C::FN, j = b % C::FN;
            if constexpr (j == 0 && !FULL) {
                const int row = trow(i);
                rmask = __ballot(row < P.M && row_active(args, row));
            }
            f32x4 xv[4];
            transpose_block(wstage, xraw[b % PD], xv);
            static_for<0, 4>([&](auto G) PCD_INLINE {
                constexpr int g = decltype(G)::value;
                f32x4 mn;
                if (folded) {
                    static_for<0, 4>([&](auto K) PCD_INLINE {
                        constexpr int k = decltype(K)::value;
                        mn[k] = xv[g][k] + eta * acc[i][j][4 * g + k];
                    });
                } else {
                    static_for<0, 4>([&](auto K) PCD_INLINE {
                        constexpr int k = decltype(K)::value;
                        const float x = xv[g][k];
                        float grad = -acc[i][j][4 * g + k];
                        if (lam > 0.f) grad += lam * (x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f));
                        mn[k] = x - eta * grad;
                    });
                }
                stage_group<4>(wstage, g, mn, PackOp<OP>{});
                if (P.mop) stage_group<OPB>(wstage2, g, mn, PackOp<OP>{});
            });
            const int brow = row0 + wm * C::WTM + i * 32, bcol = col0 + wn * C::WTN + j * 32;
            if (writer) flush_block<4, GNT>(wstage, P.m, ldo, brow, bcol, rmask, P.N, FULL || full, ntst);
            if (P.mop && writer) flush_block<OPB, GNT>(wstage2, P.mop, ldo, brow, bcol, rmask, P.N, FULL || full, ntst);
            next_operands<b, PD, NB>(load_block);
            __builtin_amdgcn_sched_barrier(0);
        });
        };
        if constexpr (C::BIG) {
            const bool gnt = ntst && ntld;
            if (full) {
                if (gnt) update(std::true_type{}, std::true_type{});
                else update(std::true_type{}, std::false_type{});
            } else {
                if (gnt) update(std::false_type{}, std::true_type{});
                else update(std::false_type{}, std::false_type{});
            }
        } else {
            update(std::false_type{}, std::false_type{});
        }
    } else if constexpr (EPI == EPI_FFG) {
        if (!writer) return;   // no barrier follows
        static_for<0, C::FM>([&](auto I) PCD_INLINE {
            constexpr int i = decltype(I)::value;
            static_for<0, C::FN>([&](auto J) PCD_INLINE {
                constexpr int j = decltype(J)::value;
                __builtin_amdgcn_sched_barrier(0);  // keep each block's epilogue to itself
                const int col = col_of(j);
                if (col < P.N) {
                    const float bj = gld(P.bias + col);
                    static_for<0, 16>([&](auto R) PCD_INLINE {
                        constexpr int r = decltype(R)::value;
                        const int row = row_of(i, r);
                        if (row < P.M) {
                            const size_t idx = (size_t)row * ldo + col;
                            const float y = act_f(args.act, acc[i][j][r] + bj);
                            gst(P.m + idx, y);
                            if (P.dout) OpTraits<OP>::store(P.dout, idx, y);
                        }
                    });
                }
            });
        });
    } else {  // EPI_PLAIN: C = alpha acc + beta C
        if (!writer) return;   // no barrier follows
        const float alpha = args.alpha, beta = args.beta;
        // whole tiles of an output too large to stay in the caches store non-temporally
        auto put = [&](float* p, float v) PCD_INLINE {
            if (ntst) __builtin_nontemporal_store(v, p);
            else gst(p, v);
        };
        static_for<0, C::FM>([&](auto I) PCD_INLINE {
            constexpr int i = decltype(I)::value;
            static_for<0, C::FN>([&](auto J) PCD_INLINE {
                constexpr int j = decltype(J)::value;
                __builtin_amdgcn_sched_barrier(0);  // keep each block's epilogue to itself
                if (full) {
                    if (beta != 0.f) {
                        float cv[16];
                        static_for<0, 16>([&](auto R) PCD_INLINE {
                            constexpr int r = decltype(R)::value;
                            cv[r] = gld(P.m + base_of(i, j) + rstep(r));
                        });
                        static_for<0, 16>([&](auto R) PCD_INLINE {
                            constexpr int r = decltype(R)::value;
                            put(P.m + base_of(i, j) + rstep(r), alpha * acc[i][j][r] + beta * cv[r]);
                        });
                    } else {
                        static_for<0, 16>([&](auto R) PCD_INLINE {
                            constexpr int r = decltype(R)::value;
                            put(P.m + base_of(i, j) + rstep(r), alpha * acc[i][j][r]);
                        });
                    }
                } else {
                    const int col = col_of(j);
                    if (col < P.N) {
                        static_for<0, 16>([&](auto R) PCD_INLINE {
                            constexpr int r = decltype(R)::value;
                            const int row = row_of(i, r);
                            if (row < P.M) {
                                const size_t idx = (size_t)row * ldo + col;
                                float v = alpha * acc[i][j][r];
                                if (beta != 0.f) v += beta * gld(P.m + idx);
                                gst(P.m + idx, v);
                            }
                        });
                    }
                }
            });
        });
    }
}

// One phase launch: workgroup b runs virtual block b.  `set` is the first
// kernel argument, so it sits at offset 0 of the kernarg segment: the problems
// are indexed there (scalar loads from constant memory) instead of being
// copied to scratch.
template <typename OP, int BM, int BN, int EPI, bool WD = false>
__global__ void __launch_bounds__((TileCfg<BM, BN, OpTraits<OP>::bytes, WD>::NT),
                                  (TileCfg<BM, BN, OpTraits<OP>::bytes, WD>::OCC))
phase_kernel(const ProblemSet set, const PhaseArgs args) {
    __shared__ __attribute__((aligned(16))) char smem[phase_smem_bytes<OP, BM, BN, WD>()];
    phase_unit<OP, BM, BN, EPI, WD>((KProblem*)__builtin_amdgcn_kernarg_segment_ptr(), set.n, args, blockIdx.x,
                                    gridDim.x, smem);
}

// ------------------------------------------------------- persistent settling

// Grid barrier of a persistent launch.  `count` starts at zero and counts
// arrivals over all barriers of the launch; `error` is set by a barrier that
// gave up.
struct GridSync {
    int* count;
    int* error;
    int spin_limit;   // polls of the arrival count before a barrier gives up
};

// The k-th barrier (k from 1) of `nw` workgroups.  Every global write a
// workgroup made before it is visible to every workgroup after it: each wave
// waits for its own stores, the workgroup barrier joins the waves, thread 0's
// device-scope fence writes them back past its XCD's L2 before the arrival is
// counted, and its fence after the wait drops the CU's and the XCD's stale
// lines before any wave reads again.  The count is read with device-scope
// atomics (coherent across the XCDs).  A barrier that polls spin_limit times
// without seeing all arrivals (or sees another's give-up) sets *error and
// returns false; the caller then leaves the kernel, so every wave exits
// normally.
__device__ __forceinline__ bool grid_barrier(const GridSync& g, int k, int nw, int* ok) {
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        __hip_atomic_fetch_add(g.count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int target = k * nw;
        int good = 1;
        for (int spins = 0;; ++spins) {
            if (__hip_atomic_load(g.count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
            if (spins >= g.spin_limit || __hip_atomic_load(g.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                __hip_atomic_store(g.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                good = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __threadfence();
        *ok = good;
    }
    __syncthreads();
    return *ok != 0;
}

// Everything one persistent settling needs, passed as the kernel's argument:
// both phases' problems (first, so the kernel indexes them in the kernarg
// segment as a phase launch does), the phases' arguments, their virtual
// grids, the step count and the barrier.
constexpr int kMaxPersistProblems = 6;
struct PersistArgs {
    Problem err_p[kMaxPersistProblems];
    Problem upd_p[kMaxPersistProblems];
    PhaseArgs err, upd;          // the phases' arguments; t is set per step
    int err_n, upd_n;            // problems per phase
    int err_grid, upd_grid;      // virtual blocks per phase (a phase launch's grid)
    int steps;
    GridSync sync;
};

// The T-step loop of a settling in one launch: every step runs all virtual
// blocks of the error phase, a grid barrier, all of the update phase, a grid
// barrier.  Workgroup w runs virtual blocks w, w + nw, ... of each phase (nw a
// multiple of the XCD count, so that a virtual block shares an XCD with the
// blocks its phase launch would have put beside it).  The units are the phase
// kernels' own, so a settling computes exactly what the per-phase launches
// compute.  The launch must be cooperative: every workgroup resident at once.
static_assert(offsetof(PersistArgs, err_p) == 0, "the problems lead the kernel argument");
template <typename OP, int BM, int BN>
__global__ void __launch_bounds__((TileCfg<BM, BN>::NT), 1) persistent_relax_kernel(const PersistArgs pa) {
    __shared__ __attribute__((aligned(16))) char smem[phase_smem_bytes<OP, BM, BN>()];
    __shared__ int ok;
    // `pa` is the only kernel argument: its problem arrays sit in the kernarg segment
    KProblem* err_p = (KProblem*)__builtin_amdgcn_kernarg_segment_ptr();
    KProblem* upd_p = err_p + kMaxPersistProblems;
    const int w = blockIdx.x, nw = gridDim.x;
    int k = 0;
    for (int t = 0; t < pa.steps; ++t) {
        PhaseArgs a = pa.err;
        a.t = t;
        for (int v = w; v < pa.err_grid; v += nw) {
            phase_unit<OP, BM, BN, EPI_ERROR>(err_p, pa.err_n, a, v, pa.err_grid, smem);
            __syncthreads();   // the next unit's loads reuse the LDS this one's epilogue read
        }
        if (!grid_barrier(pa.sync, ++k, nw, &ok)) return;
        PhaseArgs u = pa.upd;
        u.t = t;
        for (int v = w; v < pa.upd_grid; v += nw) {
            phase_unit<OP, BM, BN, EPI_UPDATE>(upd_p, pa.upd_n, u, v, pa.upd_grid, smem);
            __syncthreads();
        }
        if (!grid_barrier(pa.sync, ++k, nw, &ok)) return;
    }
}

}  // namespace pcd
