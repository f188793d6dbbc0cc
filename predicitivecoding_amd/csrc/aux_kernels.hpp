// aux_kernels.hpp -- the small kernels around the phase GEMMs: zero fill,
// operand packing and the ragged early-exit decision.  Included by the host
// translation unit only (each definition here must exist once in the library).
#pragma once
#include "pc_kernels.hpp"

namespace pcd {


// Zero-fill of n 16-byte units (used inside captured graphs instead of
// hipMemsetAsync).
__global__ void zero_kernel(u32x4* __restrict__ p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = u32x4{0u, 0u, 0u, 0u};
}

// Zero-fill of up to kZeroSegs buffers (n[k] 16-byte units at p[k]) in one
// launch: the free states a settling starts from, every layer in one node.
constexpr int kZeroSegs = 32;
struct ZeroSegs {
    u32x4* p[kZeroSegs];
    size_t n[kZeroSegs];
    int count;
};
__global__ void zero_segs_kernel(const ZeroSegs z) {
    const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (int k = 0; k < z.count; ++k) {
        u32x4* p = z.p[k];
        for (size_t i = i0; i < z.n[k]; i += stride) p[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

// Pack a row-major [rows x cols] matrix (optionally read transposed: the
// physical source is then [cols x rows]) into a zero-padded [prow x pcol]
// buffer of the operand type whose rows are `ldd` elements apart (ldd >= pcol;
// the columns past pcol are left alone).  An fp32 source is rounded to the
// operand type; a 16-bit source of the operand's own type is copied bit for
// bit.  A workgroup moves 64 x 64 tiles through LDS, so the source reads and
// the destination writes are both row-contiguous whichever way the source is
// read (one element per thread straight across a transpose reads one element
// per 2-byte segment of a row).
template <typename OP>
__global__ void __launch_bounds__(256) pack_kernel(const void* __restrict__ src, int src_is_f32, int rows, int cols,
                                                   int trans, void* __restrict__ dst, int prow, int pcol, int ldd) {
    __shared__ uint32_t tile[64][65];   // raw bits: fp32 values or 16-bit codes; 65 words a row, conflict-free
    // Thread t moves 4 consecutive elements of a row: row t/16 (+16, +32, +48), elements 4 (t%16) .. +3.
    const int q4 = (threadIdx.x & 15) * 4, qr = threadIdx.x >> 4;
    const int c0 = blockIdx.x * 64, tiles_y = (prow + 63) / 64;
    // the physical source: [rows x cols], or [cols x rows] read transposed
    const int srows = trans ? cols : rows, scols = trans ? rows : cols;
    // 4-element groups are 8- or 16-byte aligned where the row length and the base pointer allow it
    const bool vec_src = (scols & 3) == 0 && ((uintptr_t)src & (src_is_f32 ? 15 : 7)) == 0;
    const bool vec_dst = (ldd & 3) == 0 && ((uintptr_t)dst & (OpTraits<OP>::bytes * 4 - 1)) == 0;
    for (int by = blockIdx.y; by < tiles_y; by += gridDim.y) {
        const int r0 = by * 64;
        const int sr0 = trans ? c0 : r0, sc0 = trans ? r0 : c0;   // the tile's origin in the physical source
#pragma unroll
        for (int i = qr; i < 64; i += 16) {
            const int sr = sr0 + i, sc = sc0 + q4;
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            if (sr < srows) {
                const size_t at = (size_t)sr * scols + sc;
                if (vec_src && sc + 3 < scols) {
                    if (src_is_f32) {
                        const u32x4 v = *(const u32x4*)((const float*)src + at);
                        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
                    } else {
                        const u32x2 v = *(const u32x2*)((const uint16_t*)src + at);
                        w[0] = v[0] & 0xFFFFu; w[1] = v[0] >> 16; w[2] = v[1] & 0xFFFFu; w[3] = v[1] >> 16;
                    }
                } else {
                    for (int k = 0; k < 4; ++k)
                        if (sc + k < scols)
                            w[k] = src_is_f32 ? __float_as_uint(((const float*)src)[at + k]) : ((const uint16_t*)src)[at + k];
                }
            }
            // physical (i, q4 + k) is logical (i, q4 + k), or (q4 + k, i) read transposed
            for (int k = 0; k < 4; ++k) {
                if (trans) tile[q4 + k][i] = w[k];
                else tile[i][q4 + k] = w[k];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = qr; i < 64; i += 16) {
            const int r = r0 + i, c = c0 + q4;
            if (r >= prow || c >= pcol) continue;
            const size_t at = (size_t)r * ldd + c;
            uint32_t w[4];
            for (int k = 0; k < 4; ++k) w[k] = tile[i][q4 + k];
            if (vec_dst && c + 3 < pcol) {
                if (src_is_f32) {
                    const f32x4 v = {__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]),
                                     __uint_as_float(w[3])};
                    if constexpr (OpTraits<OP>::bytes == 4) *(f32x4*)((float*)dst + at) = v;
                    else *(u32x2*)((uint16_t*)dst + at) = OpTraits<OP>::pack4(v);
                } else {
                    *(u32x2*)((uint16_t*)dst + at) = u32x2{w[0] | (w[1] << 16), w[2] | (w[3] << 16)};
                }
            } else {
                for (int k = 0; k < 4 && c + k < pcol; ++k) {
                    if (src_is_f32) OpTraits<OP>::store(dst, at + k, __uint_as_float(w[k]));
                    else ((uint16_t*)dst)[at + k] = (uint16_t)w[k];
                }
            }
        }
        __syncthreads();   // the next tile row reuses `tile`
    }
}

// Fragment-major copy of a 16-bit operand [rows x cols] with rows `ld`
// elements apart (rows a multiple of 32, cols of 16): the 16-byte unit at
// dst[(rb * cols/16 + kc) * 64 + lane] holds row rb*32 + lane%32, elements
// kc*16 + 8*(lane/32) .. +7, i.e. lane `lane`'s operand of a 32 x 32 x 16
// MFMA over rows rb*32.. and K chunk kc.  A wave then reads one fragment as
// 1 KB of contiguous memory.
__global__ void frag_pack_kernel(const u32x4* __restrict__ src, int ld, int rows, int cols, u32x4* __restrict__ dst) {
    const int kcs = cols / 16;
    const size_t n = (size_t)(rows / 32) * kcs * 64;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % 64);
        const size_t f = i / 64;
        const int kc = (int)(f % kcs), rb = (int)(f / kcs);
        const int r = rb * 32 + lane % 32;
        dst[i] = src[((size_t)r * ld + (size_t)kc * 16 + 8 * (lane / 32)) / 8];
    }
}

// pack_kernel over `batch` matrices stored back to back: item i of src is the
// [rows x cols] matrix (or [cols x rows] read transposed) at src + i * rows *
// cols, packed into the zero-padded [prow x pcol] buffer at dst + i * prow *
// pcol (row pitch pcol).
template <typename OP>
__global__ void pack_batched_kernel(const void* __restrict__ src, int src_is_f32, int batch, int rows, int cols,
                                    int trans, void* __restrict__ dst, int prow, int pcol) {
    const size_t per = (size_t)prow * pcol, n = per * batch, src_per = (size_t)rows * cols;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (size_t)gridDim.x * blockDim.x) {
        const size_t item = k / per, e = k % per;
        const int r = (int)(e / pcol), c = (int)(e % pcol);
        const bool inside = r < rows && c < cols;
        const size_t s = item * src_per + (trans ? (size_t)c * rows + r : (size_t)r * cols + c);
        if (src_is_f32) {
            OpTraits<OP>::store(dst, k, inside ? ((const float*)src)[s] : 0.f);
        } else {
            // 16-bit source of the operand's own type: copy the bits
            ((uint16_t*)dst)[k] = inside ? ((const uint16_t*)src)[s] : (uint16_t)0;
        }
    }
}

// Weight formats of a LayerSerializer record (Model/LayerSerializer.cs:19-36).
enum RecordKind { REC_F32 = 0, REC_F16 = 1, REC_BF16 = 2, REC_I8 = 3 };

// Pack the [rows x cols] weights of a record (optionally read transposed) into
// a zero-padded [prow x pcol] operand buffer (row pitch pcol).  Values are
// widened to fp32 as the reference's Deserialize does -- Half and bf16 exactly,
// int8 as (q - z) * s with the row's scale and zero point (:299-312) -- and
// then stored in the operand type, which keeps a record of the operand's own
// 16-bit format bit for bit.
template <typename OP>
__global__ void pack_record_kernel(const void* __restrict__ src, int kind, const float* __restrict__ scales,
                                   const int8_t* __restrict__ zeros, int rows, int cols, int trans,
                                   void* __restrict__ dst, int prow, int pcol) {
    const size_t n = (size_t)prow * pcol;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / pcol), c = (int)(i % pcol);
        float v = 0.f;
        if (r < rows && c < cols) {
            // logical (r, c) of op(W); W itself is [rows x cols], or [cols x rows] read transposed
            const int pr = trans ? c : r, pc = trans ? r : c;
            const size_t s = (size_t)pr * (trans ? rows : cols) + pc;
            switch (kind) {
            case REC_F32: v = ((const float*)src)[s]; break;
            case REC_BF16: v = __uint_as_float((uint32_t)((const uint16_t*)src)[s] << 16); break;
            case REC_F16: v = (float)__builtin_bit_cast(_Float16, ((const uint16_t*)src)[s]); break;
            default: v = (float)((int)((const int8_t*)src)[s] - (int)zeros[pr]) * scales[pr]; break;
            }
        }
        OpTraits<OP>::store(dst, i, v);
    }
}

// Ragged early exit, one workgroup per request, between the error and the
// update phase of step t: sums the request's row energies, records them and
// decides whether step t is its last (Network.cs:895-905).
__global__ void exit_kernel(const float* __restrict__ part, int ldp, int nslots, const int* __restrict__ row_offsets,
                            int* __restrict__ done_at, float* __restrict__ prev_energy, float* __restrict__ last_energy,
                            int t, int rule, float thr) {
    const int r = blockIdx.x;
    if (t >= done_at[r]) return;  // uniform over the workgroup
    const int r0 = row_offsets[r], r1 = row_offsets[r + 1];
    float s = 0.f;
    for (int row = r0 + threadIdx.x; row < r1; row += blockDim.x)
        s += sum_slots(part, ldp, nslots, row);
    __shared__ float red[256];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float e = red[0];
        const float prev = prev_energy[r];
        bool stop = false;
        if (rule == 1) stop = thr > 0.f && t > 0 && (prev - e < thr * fmaxf(prev, 1e-12f));
        else if (rule == 2) stop = e / (float)(r1 - r0) < thr;
        last_energy[r] = e;
        prev_energy[r] = e;
        if (stop) done_at[r] = t + 1;
    }
}

// exit_kernel for calls whose every request is one row (request r is row r):
// one thread per request.  The same sum and the same decision as exit_kernel
// (whose tree over one row's value only adds zeros).
__global__ void exit_rows_kernel(const float* __restrict__ part, int ldp, int nslots, int requests,
                                 int* __restrict__ done_at, float* __restrict__ prev_energy,
                                 float* __restrict__ last_energy, int t, int rule, float thr) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < requests; r += gridDim.x * blockDim.x) {
        if (t >= done_at[r]) continue;
        const float e = sum_slots(part, ldp, nslots, r);
        const float prev = prev_energy[r];
        bool stop = false;
        if (rule == 1) stop = thr > 0.f && t > 0 && (prev - e < thr * fmaxf(prev, 1e-12f));
        else if (rule == 2) stop = e < thr;
        last_energy[r] = e;
        prev_energy[r] = e;
        if (stop) done_at[r] = t + 1;
    }
}

// Tables of a call whose every request is one row (request r is row r):
// row -> request, row offsets, step budgets, exit state.
__global__ void row_request_tables_kernel(int* __restrict__ row_req, int* __restrict__ offsets,
                                          int* __restrict__ done_at, float* __restrict__ prev_energy,
                                          float* __restrict__ last_energy, int rows, int steps) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r <= rows; r += gridDim.x * blockDim.x) {
        offsets[r] = r;
        if (r < rows) {
            row_req[r] = r;
            done_at[r] = steps;
            prev_energy[r] = 0.f;
            last_energy[r] = 0.f;
        }
    }
}

// Adaptive classification (Network.PredictAdaptive, Network.cs:803-840): row
// b * classes + c settled candidate c of sample b for done_at steps and ended
// at energy e.  The class is the first c with the smallest energy (below
// float.MaxValue, :822); the winner's re-run (:826-828) repeats its settling,
// so its energy is its candidate's and its steps count twice.  Each output is
// written where its pointer is set.
__global__ void adaptive_argmin_kernel(const float* __restrict__ e, const int* __restrict__ done_at, int batch,
                                       int classes, float* __restrict__ table, int* __restrict__ steps_table,
                                       int* __restrict__ cls, float* __restrict__ best, int* __restrict__ steps_used) {
    for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < batch; b += gridDim.x * blockDim.x) {
        float be = 3.402823466e38f;   // float.MaxValue
        int bc = 0, total = 0;
        for (int c = 0; c < classes; ++c) {
            const size_t r = (size_t)b * classes + c;
            const float v = e[r];
            const int k = done_at[r];
            if (table) table[r] = v;
            if (steps_table) steps_table[r] = k;
            total += k;
            if (v < be) { be = v; bc = c; }
        }
        const size_t w = (size_t)b * classes + bc;
        if (cls) cls[b] = bc;
        if (best) best[b] = e[w];
        if (steps_used) steps_used[b] = total + done_at[w];
    }
}

// Ragged: the row tiles of bm rows that hold a row still running at step t
// (a row of request r runs while t < done_at[r]), listed in increasing order,
// and their number.  One workgroup of kActTilesThreads threads; at most
// kMaxActTiles row tiles.  Requests own the contiguous row ranges
// [row_offsets[r], row_offsets[r + 1]).
constexpr int kActTilesThreads = 1024;
constexpr int kMaxActTiles = 16384;
__global__ void __launch_bounds__(kActTilesThreads)
active_tiles_kernel(const int* __restrict__ row_offsets, const int* __restrict__ done_at, int requests, int rows,
                    int bm, int t, int* __restrict__ list, int* __restrict__ count) {
    __shared__ unsigned char live[kMaxActTiles];
    __shared__ int sums[kActTilesThreads];
    const int tid = threadIdx.x;
    const int ntiles = min((rows + bm - 1) / bm, kMaxActTiles);
    for (int i = tid; i < ntiles; i += kActTilesThreads) live[i] = 0;
    __syncthreads();
    for (int r = tid; r < requests; r += kActTilesThreads) {
        const int r0 = row_offsets[r], r1 = min(row_offsets[r + 1], rows);
        if (r1 > r0 && t < done_at[r])
            for (int i = r0 / bm; i <= (r1 - 1) / bm && i < ntiles; ++i) live[i] = 1;
    }
    __syncthreads();
    // Thread tid owns the contiguous tiles [tid * per, (tid + 1) * per): count,
    // scan the counts over the workgroup, then write the owned entries.
    const int per = (ntiles + kActTilesThreads - 1) / kActTilesThreads;
    const int lo = min(tid * per, ntiles), hi = min(lo + per, ntiles);
    int mine = 0;
    for (int i = lo; i < hi; ++i) mine += live[i];
    sums[tid] = mine;
    __syncthreads();
    for (int d = 1; d < kActTilesThreads; d <<= 1) {
        const int add = tid >= d ? sums[tid - d] : 0;
        __syncthreads();
        sums[tid] += add;
        __syncthreads();
    }
    int at = sums[tid] - mine;
    for (int i = lo; i < hi; ++i)
        if (live[i]) list[at++] = i;
    if (tid == kActTilesThreads - 1) count[0] = sums[tid];
}

// Row energies of a step from the per-slot partials when no update-phase
// launch is there to reduce them (every free layer clamped).
__global__ void energy_rows_kernel(const float* __restrict__ part, int ldp, int nslots, float* __restrict__ out,
                                   int rows) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
        out[r] = sum_slots(part, ldp, nslots, r);
    }
}

// Layer-0 rows of a classification batch: row r is sample r / classes of x0
// ([batch x cols], packed), copied into the fp32 state [rows x ld].
__global__ void replicate_rows_kernel(const float* __restrict__ x0, int cols, int classes, int rows,
                                      float* __restrict__ dst, int ld) {
    const size_t n = (size_t)rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        dst[(size_t)r * ld + c] = x0[(size_t)(r / classes) * cols + c];
    }
}

// Clamped top rows: from src ([rows x cols], packed) or, with src null, the
// one-hot of class r % cols (ClassEnergies' candidate label), written to the
// fp32 state [rows x ld] and, when dst_op is set, to its operand-type copy.
// Columns cols..ld-1 are written zero.
template <typename OP>
__global__ void top_rows_kernel(const float* __restrict__ src, int cols, int rows, float* __restrict__ dst,
                                void* __restrict__ dst_op, int ld) {
    const size_t n = (size_t)rows * ld;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / ld), c = (int)(i % ld);
        float v = 0.f;
        if (c < cols) v = src ? src[(size_t)r * cols + c] : (c == r % cols ? 1.f : 0.f);
        dst[i] = v;
        if (dst_op) OpTraits<OP>::store(dst_op, i, v);
    }
}

// Minimum-energy class per sample (Network.PredictCore, Network.cs:385-396):
// the first class with the smallest energy.  e holds the [batch x classes]
// last-step energies; the per-class table, the class and its energy are written
// where the pointers are set.
__global__ void class_argmin_kernel(const float* __restrict__ e, int batch, int classes, float* __restrict__ table,
                                    int* __restrict__ cls, float* __restrict__ best) {
    for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < batch; b += gridDim.x * blockDim.x) {
        float be = 3.402823466e38f;   // float.MaxValue
        int bc = 0;
        for (int c = 0; c < classes; ++c) {
            const float v = e[(size_t)b * classes + c];
            if (table) table[(size_t)b * classes + c] = v;
            if (v < be) { be = v; bc = c; }
        }
        if (cls) cls[b] = bc;
        // the winner's energy as the reference's re-run of the winning class returns it
        if (best) best[b] = e[(size_t)b * classes + bc];
    }
}

// Bias step of the learning rule (Layer.cs:327): b[i] += eta_w * sum over the
// batch rows of D[r][i], rows summed in order.
// D is in the operand type (16-bit models keep it 16-bit).
template <typename OP>
__global__ void bias_update_kernel(const void* __restrict__ d, int ld, int rows, int cols, float* __restrict__ bias,
                                   float eta_w) {
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x) {
        // Rows eight at a time: the loads go out together, the adds stay in
        // row order (the same sum as one row after another).
        float s = 0.f;
        int r = 0;
        for (; r + 8 <= rows; r += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = OpTraits<OP>::load(d, (size_t)(r + k) * ld + c);
#pragma unroll
            for (int k = 0; k < 8; ++k) s += v[k];
        }
        for (; r < rows; ++r) s += OpTraits<OP>::load(d, (size_t)r * ld + c);
        bias[c] += eta_w * s;
    }
}

// The learning step's weight and bias update for a batch of at most a few
// hundred rows, every layer
// in one launch: W_l = beta W_l + alpha D_l^T M_l (K = the batch rows, summed
// in row order on the VALU), b_l += eta_w * (column sums of D_l, rows in
// order), and the refreshed operand copies W_l^T and, for 16-bit models,
// W_l, rounded as the upload rounds them.  Workgroup b runs one 32 x 32 block
// of one layer's W (blocks counted layer after layer); lane t owns rows
// i0 + 2 (t % 16) + {0, 1} and columns j0 + 2 (t / 16) + {0, 1}, with
// 64-row chunks of its D and M columns staged in LDS.
constexpr int kHebbLayers = 16;   // layers per launch
struct HebbLayer {
    const void* d;     // D_l [batch x ldd], operand type
    const float* m;    // M_l [batch x ldm]
    float* w;          // W_l, fp32 (the model's weights or 16-bit models' masters) [lo x ldw]
    void* w16;         // 16-bit copy of W_l [lo x ldw], or null (fp32 models)
    void* wt;          // W_l^T in the operand type [sz x ldwt]
    float* bias;       // b_l [lo]
    int ldd, ldm, ldw, ldwt;
    int lo, sz;        // rows and columns of W_l
    int blocks;        // ceil(lo / 32) * ceil(sz / 32)
};
struct HebbSet {
    HebbLayer l[kHebbLayers];
    int n, batch;
    float alpha, beta, eta_w;
};
template <typename OP>
__global__ void __launch_bounds__(256) hebbian_small_kernel(const HebbSet set) {
    __shared__ float sd[64][33], sm[64][33];
    int b = blockIdx.x, q = 0;
    while (q < set.n && b >= set.l[q].blocks) b -= set.l[q++].blocks;
    if (q >= set.n) return;
    const HebbLayer& L = set.l[q];
    const int nbj = (L.sz + 31) / 32;
    const int i0 = (b / nbj) * 32, j0 = (b % nbj) * 32;
    const int t = threadIdx.x, ti = t % 16, tj = t / 16;
    float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}}, bs[2] = {0.f, 0.f};
    const bool bias_lane = j0 == 0 && tj == 0;
    for (int r0 = 0; r0 < set.batch; r0 += 64) {
        const int nr = min(64, set.batch - r0);
        __syncthreads();
        for (int e = t; e < 64 * 32; e += 256) {
            const int r = e / 32, c = e % 32;
            const bool ok = r < nr;
            sd[r][c] = ok && i0 + c < L.lo ? OpTraits<OP>::load(L.d, (size_t)(r0 + r) * L.ldd + i0 + c) : 0.f;
            sm[r][c] = ok && j0 + c < L.sz ? L.m[(size_t)(r0 + r) * L.ldm + j0 + c] : 0.f;
        }
        __syncthreads();
        for (int r = 0; r < nr; ++r) {
            const float d0 = sd[r][2 * ti], d1 = sd[r][2 * ti + 1];
            const float m0 = sm[r][2 * tj], m1 = sm[r][2 * tj + 1];
            acc[0][0] = fmaf(d0, m0, acc[0][0]);
            acc[0][1] = fmaf(d0, m1, acc[0][1]);
            acc[1][0] = fmaf(d1, m0, acc[1][0]);
            acc[1][1] = fmaf(d1, m1, acc[1][1]);
            if (bias_lane) {
                bs[0] += d0;
                bs[1] += d1;
            }
        }
    }
    for (int a = 0; a < 2; ++a) {
        const int i = i0 + 2 * ti + a;
        if (i >= L.lo) continue;
        if (bias_lane) L.bias[i] += set.eta_w * bs[a];
        for (int c = 0; c < 2; ++c) {
            const int j = j0 + 2 * tj + c;
            if (j >= L.sz) continue;
            float* wp = L.w + (size_t)i * L.ldw + j;
            const float v = set.alpha * acc[a][c] + set.beta * *wp;
            *wp = v;
            if (L.w16) OpTraits<OP>::store(L.w16, (size_t)i * L.ldw + j, v);
            OpTraits<OP>::store(L.wt, (size_t)j * L.ldwt + i, v);
        }
    }
}

// Rows of a ragged call between the caller's packing and the settling order:
// gather dst[i] = src[perm[i]], scatter dst[perm[i]] = src[i], `cols` floats
// per row.  perm is a permutation of [0, rows).
__global__ void permute_rows_kernel(const float* __restrict__ src, int lds, float* __restrict__ dst, int ldd,
                                    const int* __restrict__ perm, int rows, int cols, int gather) {
    const size_t n = (size_t)rows * cols;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(e / cols), c = (int)(e % cols);
        const int p = perm[i];
        if (gather) dst[(size_t)i * ldd + c] = src[(size_t)p * lds + c];
        else dst[(size_t)p * ldd + c] = src[(size_t)i * lds + c];
    }
}

}  // namespace pcd
