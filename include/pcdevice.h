/*
 * pcdevice.h -- C ABI of libpcdevice_hip, the MI355X (gfx950) implementation
 * of the batched predictive-coding relaxation of matteofabbri/PredicitiveCoding
 * (PredictiveCoding.Device/BatchedPcForward.cs) and of the device runtime
 * calls that path makes.
 *
 * Conventions, following the reference's P/Invoke layer
 * (PredictiveCoding.Device/Interop/Cuda.cs:16-50, Cublas.cs:25-59):
 *   - every entry point is cdecl and returns an int status (0 = success); the
 *     codes are the reference's DeviceStatus enum (Interop/CudaStatus.cs:7-19);
 *   - handles come back through out-pointers;
 *   - host buffers are read during the call only and never retained
 *     (DeviceTensor.cs:94-120);
 *   - device pointers are HIP device memory (pcd_malloc_async, or any other
 *     HIP allocation in the same process);
 *   - work is queued on the given stream (NULL = the device's null stream)
 *     and is complete only after a synchronisation.
 * Thread safety: distinct streams may be used from distinct threads; a model
 * handle is immutable after creation; the per-call scratch belongs to the
 * (model, stream) pair.  A call that records its settling into a HIP graph
 * (the first call of a shape on a stream) and the library's synchronous copies
 * (pcd_memcpy, weight uploads) exclude each other, because HIP fails a
 * legacy-stream operation made while any stream of the process is recording;
 * a caller's own legacy-stream calls made meanwhile are not covered.
 */
#ifndef PCDEVICE_H
#define PCDEVICE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DeviceStatus, Interop/CudaStatus.cs:7-19 (CudaError/CublasError carry HIP
 * runtime and GEMM failures here). */
enum pcd_status {
    PCD_SUCCESS = 0,
    PCD_NOT_INITIALIZED = 1,
    PCD_NO_DEVICE = 2,
    PCD_OUT_OF_MEMORY = 3,
    PCD_INVALID_VALUE = 4,
    PCD_HIP_ERROR = 5,
    PCD_GEMM_ERROR = 6,
    PCD_COLLECTIVE_ERROR = 7, /* unused: no multi-GPU path */
    PCD_NOT_SUPPORTED = 8,
    PCD_UNKNOWN = 100
};

/* MemcpyKind, Interop/Cuda.cs:6 */
enum pcd_memcpy_kind {
    PCD_HOST_TO_HOST = 0,
    PCD_HOST_TO_DEVICE = 1,
    PCD_DEVICE_TO_HOST = 2,
    PCD_DEVICE_TO_DEVICE = 3,
    PCD_MEMCPY_DEFAULT = 4
};

/* ActivationType, PredicitiveCoding/Core/Activation.cs:19-25, extended with
 * the tanh-approximation GELU used throughout the reference
 * (PredictiveCoding.LLM/Model/Layers.cs:42-50). */
enum pcd_activation {
    PCD_ACT_LINEAR = 0,
    PCD_ACT_TANH = 1,
    PCD_ACT_RELU = 2,
    PCD_ACT_SIGMOID = 3,
    PCD_ACT_GELU = 4
};

/* Storage/operand type of the weights and of the GEMM operands.
 *   PCD_F32   fp32 everything (InferGetTopBatch, mixed = false)
 *   PCD_F16   weights and both GEMM operands rounded to fp16, fp32 accumulate,
 *             fp32 states/errors/energy (the reference's mixed = true,
 *             Gemm.cs:44-60, CudaGemmProvider.cs:150-202)
 *   PCD_BF16  as PCD_F16 with bf16 round-to-nearest-even
 *             (TensorUtils.cs:379-401) */
enum pcd_dtype { PCD_F32 = 0, PCD_BF16 = 1, PCD_F16 = 2 };

/* Early-exit rule of the ragged entry point.
 *   PCD_EXIT_NONE      run every request for its full step budget
 *   PCD_EXIT_RELATIVE  Network.SettleAdaptive (Network.cs:876-907): stop after
 *                      a step once prev - E < thr * max(prev, 1e-12); the
 *                      first step never exits
 *   PCD_EXIT_ABSOLUTE  stop after a step once E / rows_of_request < thr
 * E is the request's energy summed over its rows, read before the update of
 * the step (Network.cs:939-945 over Layer.cs:437-450). */
enum pcd_exit_rule { PCD_EXIT_NONE = 0, PCD_EXIT_RELATIVE = 1, PCD_EXIT_ABSOLUTE = 2 };

typedef struct pcd_model pcd_model;

/* ---------------------------------------------------------------- runtime */

/* cudaGetDeviceCount, Interop/Cuda.cs:23; DeviceRuntime probing
 * (DeviceRuntime.cs:27-32,68-82): no GPU gives *count = 0 and PCD_NO_DEVICE. */
int pcd_get_device_count(int* count);
/* cudaSetDevice, Interop/Cuda.cs:24 */
int pcd_set_device(int device);
int pcd_get_device(int* device);
/* cudaDeviceSynchronize, Interop/Cuda.cs:25 */
int pcd_device_synchronize(void);
/* Text of the calling thread's last failure (empty if none). Replaces the
 * exception message NativeCheck.Ok builds (CudaStatus.cs:22-38). */
int pcd_last_error(char* buf, size_t len);
/* Library version as major*10000 + minor*100 + patch. */
int pcd_version(int* version);

/* ----------------------------------------------------------------- memory */

/* Pooled device allocation: IDeviceAllocator.Allocate/Free
 * (Allocators/IDeviceAllocator.cs:6-18) as CudaAllocator implements them
 * (Allocators/CudaAllocator.cs:32-59): power-of-two buckets of at most 32
 * cached blocks, stream-ordered allocation with a synchronous fallback. */
int pcd_malloc_async(void** ptr, size_t bytes, void* stream);
int pcd_free_async(void* ptr, void* stream);
/* Pinned host memory: CudaAllocator.AllocatePinnedHost/FreePinnedHost
 * (CudaAllocator.cs:63-84). */
int pcd_host_alloc(void** ptr, size_t bytes);
int pcd_host_free(void* ptr);
/* Releases every cached block of both pools (CudaAllocator.TrimPools). */
int pcd_trim_pools(void);
/* cudaMemcpy / cudaMemcpyAsync / cudaMemsetAsync, Interop/Cuda.cs:37-39 */
int pcd_memcpy(void* dst, const void* src, size_t bytes, int kind);
int pcd_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream);
int pcd_memset_async(void* dst, int value, size_t bytes, void* stream);

/* -------------------------------------------------------- streams, events */

/* CudaStreamManager.CreateStream/Synchronize (Streams/CudaStreamManager.cs:38-52)
 * over cudaStreamCreate/Destroy/Synchronize (Interop/Cuda.cs:42-44).  Streams
 * are created non-blocking at the default priority. */
int pcd_stream_create(void** stream);
int pcd_stream_destroy(void* stream);
int pcd_stream_synchronize(void* stream);
/* RecordEvent/WaitEvent (CudaStreamManager.cs:62-75) over the event calls of
 * Interop/Cuda.cs:45-48, plus the elapsed time between two events. */
int pcd_event_create(void** event);
int pcd_event_record(void* event, void* stream);
int pcd_event_synchronize(void* event);
int pcd_event_destroy(void* event);
int pcd_event_elapsed_ms(float* ms, void* start, void* end);

/* ------------------------------------------------------------------- GEMM */

/* Row-major C[m,n] = op(A) op(B) + beta C on device pointers, the semantics of
 * CudaGemmProvider.MatMulDeviceEx (Gemm/CudaGemmProvider.cs:82-98): op(A) is
 * A [m,k] or, with trans_a, the transpose of a physical [k,m] A (same for B).
 * With trans_a = trans_b = 0 and beta = 0 this is MatMulDevice (:62-72).
 * Operands are read where they lie when aligned and whole-tile shaped
 * (16-bit operands in either layout: a row-major B or a transposed A is
 * transposed in LDS); others
 * are packed into scratch from the library's pool. */
int pcd_gemm_f32(const float* dA, const float* dB, float* dC, int m, int k, int n,
                 int trans_a, int trans_b, float beta, void* stream);
/* bf16 operands (raw bf16 bit patterns), fp32 accumulation and fp32 C:
 * CudaGemmProvider.MatMulDeviceExBf16 (CudaGemmProvider.cs:107-127). */
int pcd_gemm_bf16(const uint16_t* dA, const uint16_t* dB, float* dC, int m, int k, int n,
                  int trans_a, int trans_b, float beta, void* stream);
/* fp16 operands: CudaGemmProvider.MatMulMixedDevice (CudaGemmProvider.cs:185-202). */
int pcd_gemm_f16(const uint16_t* dA, const uint16_t* dB, float* dC, int m, int k, int n,
                 int trans_a, int trans_b, float beta, void* stream);
/* Strided batched GEMM, CudaGemmProvider.MatMulBatchedDevice
 * (CudaGemmProvider.cs:130-141): for i < batch, row-major
 * C_i[m,n] = A_i[m,k] B_i[k,n] with A_i at dA + i*m*k, B_i at dB + i*k*n and
 * C_i at dC + i*m*n (elements); fp32 C.  The _bf16 and _f16 forms take 16-bit
 * operands (raw bit patterns) with fp32 accumulation.  Scratch for operand
 * packing comes from the library's pool. */
int pcd_gemm_f32_batched(const float* dA, const float* dB, float* dC, int batch, int m, int k, int n,
                         void* stream);
int pcd_gemm_bf16_batched(const uint16_t* dA, const uint16_t* dB, float* dC, int batch, int m, int k, int n,
                          void* stream);
int pcd_gemm_f16_batched(const uint16_t* dA, const uint16_t* dB, float* dC, int batch, int m, int k, int n,
                         void* stream);

/* --------------------------------------------------------- PC relaxation */

/* Uploads a GenerativeSnapshot (Networks/GenerativeSnapshot.cs:15-23) to the
 * current device.
 *   sizes[levels]       LayerSizes, levels >= 2
 *   W[levels-1]         host pointers; W[l-1] is W_l [sizes[l-1] x sizes[l]] row-major
 *   b[levels-1]         host pointers; b[l-1] is b_l [sizes[l-1]]
 *   precisions[levels]  scalar precision per layer (> 0)
 *   eta, act_reg        StateLearningRate, ActivityRegularization (>= 0)
 *   ffg                 UseFeedforwardGistInit
 *   dtype               enum pcd_dtype
 * The library keeps its own device copies (W and W^T in the operand dtype,
 * biases in fp32); host memory is read during the call only.  W and b may
 * both be null: the weights and biases then start at zero, for
 * pcd_pc_model_load_record to fill. */
int pcd_pc_model_create(const int* sizes, int levels, int activation, float eta, float act_reg, int ffg,
                        const float* const* W, const float* const* b, const float* precisions,
                        int dtype, pcd_model** out);
int pcd_pc_model_destroy(pcd_model* model);

/* BatchedPcForward.InferGetTopBatch (BatchedPcForward.cs:36-139): settles
 * `batch` samples for `steps` steps from zero free states, layer 0 clamped to
 * x0.  All pointers are device pointers.
 *   x0          [batch x sizes[0]]
 *   out_top     [batch x sizes[levels-1]]
 *   out_states  nullable; every layer l = 0..levels-1 as [batch x sizes[l]],
 *               concatenated in layer order
 *   out_energy  nullable; [steps x batch] per-sample energy of each step
 * Errors: PCD_INVALID_VALUE for batch < 1 ("Empty batch.", :44), steps < 1
 * (:45) or null pointers.  (The per-input length check of :55-57 is the
 * caller's, since x0 arrives packed.)  Asynchronous on `stream`. */
int pcd_pc_relax(pcd_model* model, const float* x0, int batch, int steps,
                 float* out_top, float* out_states, float* out_energy, void* stream);

/* No counterpart in the reference: pcd_pc_relax for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * pcd_pc_relax, but the call allocates nothing: its scratch (states, deltas,
 * energy partials, split-K partial tiles) lives in a library-owned device
 * array of 64 MiB per device, which each device holds until the process ends,
 * and the step loop runs as plain kernel launches (no cached graph).  A call
 * whose batch needs more scratch than that fails with PCD_INVALID_VALUE
 * before launching anything (pcd_last_error names the size).  Every call on a
 * device shares that device's array: the library runs such calls one after
 * another, whatever their streams, threads or models (each call's stream waits
 * on an event the previous call recorded, set up with the array on the first
 * call).  A call made while its stream is being captured into a graph is
 * ordered only by that graph: the caller orders the graph's replays against
 * other uses of the array.  out_energy, when given, is written in place.
 * Asynchronous on `stream`. */
int pcd_pc_relax_noalloc(pcd_model* model, const float* x0, int batch, int steps,
                         float* out_top, float* out_states, float* out_energy, void* stream);

/* Ragged request batches: request r owns rows [row_offsets[r], row_offsets[r+1])
 * of x0_packed and settles for at most steps[r] steps, leaving early by
 * exit_rule / exit_threshold (enum pcd_exit_rule) -- Network.InferAdaptive
 * (Network.cs:760-782) applied per request, all requests in one packed launch.
 * Device pointers:
 *   x0_packed   [rows x sizes[0]], rows = row_offsets[requests]
 *   out_top     [rows x sizes[levels-1]]
 * Host pointers (read or written during the call, which synchronises `stream`):
 *   row_offsets [requests+1] increasing, row_offsets[0] = 0
 *   steps       [requests]   each >= 1
 *   steps_used  [requests]   steps each request ran
 *   out_energy  [requests]   nullable; the request's energy at its last step
 */
int pcd_pc_relax_ragged(pcd_model* model, const float* x0_packed, const int* row_offsets, const int* steps,
                        int requests, int exit_rule, float exit_threshold, int* steps_used,
                        float* out_top, float* out_energy, void* stream);

/* Network.InferCore with the top clamped (Network.cs:75-111 with clampTop and a
 * label; the settling of Network.InferEnergy, :234-244): layer 0 holds x0,
 * layer levels-1 holds `top` and is never updated (Layer.cs:275), the hidden
 * layers start at zero.  Device pointers:
 *   x0          [batch x sizes[0]],  top [batch x sizes[levels-1]]
 *   out_states  nullable; every layer as in pcd_pc_relax
 *   out_energy  nullable; [steps x batch] per-sample energy of each step (the
 *               last row is InferEnergy's ComputeEnergyCore)
 * Errors as pcd_pc_relax.  Asynchronous on `stream`. */
int pcd_pc_relax_clamped(pcd_model* model, const float* x0, const float* top, int batch, int steps,
                         float* out_states, float* out_energy, void* stream);

/* Minimum-energy classification of a batch: Network.ClassEnergies
 * (Network.cs:253-278) and Network.PredictCore (:369-415) for every sample
 * at once.  Each sample is settled C = sizes[levels-1] times, the top clamped
 * to one-hot(c) and the hidden layers starting at zero (batch x C packed rows);
 * F(x, c) is the energy of the last step.  The class is the first c with the
 * smallest F (:395), and its energy is F(x, c*) (the reference re-runs the
 * winner, :400-406, which repeats the same settling).  Device pointers, each
 * nullable but not all null:
 *   x0                  [batch x sizes[0]]
 *   out_class_energies  [batch x C]   ClassEnergies
 *   out_class           [batch]       Predict
 *   out_energy          [batch]       PredictWithEnergy's energy
 * Errors as pcd_pc_relax.  Asynchronous on `stream`. */
int pcd_pc_classify(pcd_model* model, const float* x0, int batch, int steps, float* out_class_energies,
                    int* out_class, float* out_energy, void* stream);

/* Adaptive minimum-energy classification of a batch: Network.PredictAdaptive
 * (Network.cs:803-840) for every sample at once.  Each class candidate c of
 * sample b (row b * C + c, C = sizes[levels-1]) settles from zero hidden
 * states with the top clamped to one-hot(c), as SettleCandidate (:851-867),
 * for at most max_steps steps, and stops after a step once
 * prev - E < epsilon * max(prev, 1e-12) (SettleAdaptive, :876-907; never after
 * the first step; epsilon <= 0 never stops, which is pcd_pc_classify).  E(b, c)
 * is the candidate's energy at its last step; the class is the first c with
 * the smallest E; the reference re-runs the winner (:826-828), which repeats
 * its candidate's settling: its energy is E(b, c*) and its steps count twice.
 * EffortPresets.For (EffortLevel.cs:33-39) gives (max_steps, epsilon):
 * Low (10, 1e-3), Medium (30, 1e-4), High (100, 1e-5).  Device pointers, each
 * nullable but not all null:
 *   x0                  [batch x sizes[0]]
 *   out_class_energies  [batch x C]   E(b, c)
 *   out_class_steps     [batch x C]   steps candidate c of sample b ran
 *   out_class           [batch]       the class (PredictAdaptive's cls)
 *   out_energy          [batch]       its energy (energy)
 *   out_steps_used      [batch]       sum over c of the steps, plus the
 *                                     winner's again (stepsUsed)
 * Errors: PCD_INVALID_VALUE for batch < 1 ("Empty batch."), max_steps < 1,
 * a null input or no output.  Asynchronous on `stream`. */
int pcd_pc_classify_adaptive(pcd_model* model, const float* x0, int batch, int max_steps, float epsilon,
                             float* out_class_energies, int* out_class_steps, int* out_class, float* out_energy,
                             int* out_steps_used, void* stream);

/* Learning step, Network.Learn (Network.cs:139-155): settles with x0 and
 * `labels` clamped (as pcd_pc_relax_clamped), then updates every layer's
 * weights in place with Layer.UpdateWeights (Layer.cs:320-333), the last step's
 * delta_l = f'(pre_l) * e_{l-1} and the settled states:
 *   W_l += eta_w delta_l^T mu_l,  b_l += eta_w sum delta_l,  W_l -= eta_w weight_decay W_l.
 * A batch applies the sum of its samples' updates, all taken at the weights
 * the call starts from.  The hidden layers start from zero: with batch = 1
 * this is Learn on a network whose hidden states are zero (fresh, or after a
 * resetState settling).  The reference's Learn starts from the hidden states
 * the network last persisted (ReadAllLayers, :143) and persists the settled
 * ones; pcd_pc_learn_warm takes and returns them.  Device pointers:
 *   x0 [batch x sizes[0]], labels [batch x sizes[levels-1]],
 *   out_energy nullable [batch], each sample's energy at the last step.
 * A 16-bit model keeps fp32 master weights and updates those, then re-rounds
 * its operands: Network.LearnMixed (Network.cs:158-181); its delta is the
 * 16-bit value the settling's W^T GEMM consumed (the reference's per-sample
 * path keeps it fp32).  The model's weights change: no other call on the model
 * may run concurrently (any stream).
 * Asynchronous on `stream`. */
int pcd_pc_learn(pcd_model* model, const float* x0, const float* labels, int batch, int steps, float eta_w,
                 float weight_decay, float* out_energy, void* stream);

/* pcd_pc_learn with the hidden states carried as Network.Learn carries them
 * (Network.cs:139-155: ReadAllLayers restores each layer's persisted Mu,
 * InferCore resets nothing, _store.Write persists the settled Mu).  Device
 * pointers, the hidden layers l = 1..levels-2 as [batch x sizes[l]] blocks
 * concatenated in layer order:
 *   hidden_in   nullable; the states the settling starts from (null: zero)
 *   hidden_out  nullable; the settled states, to pass as the next call's
 *               hidden_in (may alias hidden_in)
 * With the same model, passing each call's hidden_out to the next reproduces
 * the reference's sequence of Learn calls on one network.  Otherwise as
 * pcd_pc_learn.  Asynchronous on `stream`. */
int pcd_pc_learn_warm(pcd_model* model, const float* x0, const float* labels, const float* hidden_in,
                      float* hidden_out, int batch, int steps, float eta_w, float weight_decay, float* out_energy,
                      void* stream);

/* Reads layer `layer`'s (1..levels-1) current weights back to host memory, as
 * Network.ExportGenerativeSnapshot copies them (Network.cs:1328-1356):
 *   W_out  nullable host [sizes[layer-1] x sizes[layer]] (16-bit models give
 *          their fp32 master weights)
 *   b_out  nullable host [sizes[layer-1]]
 * Waits for the device. */
int pcd_pc_model_get_weights(pcd_model* model, int layer, float* W_out, float* b_out);

/* Loads one LayerSerializer record (PredicitiveCoding/Model/LayerSerializer.cs:8-41,
 * the layer's persisted bytes, host memory) into the model: layer `layer`'s
 * precision and, for layer >= 1, its weights and bias, straight into the
 * device operands in the record's own format:
 *   float32, Half (flag 4), bfloat16 (flag 8): widened exactly, then stored in
 *     the operand type (a record in the operand's own 16-bit format is copied
 *     bit for bit);
 *   int8 affine per row (flag 16): dequantized on the device as
 *     (q - z) * s (ReadInt8Weights, :299-312).
 * Deserialize's checks apply: sizes must match the model ("Layer size
 * mismatch", :154-157); a record with a diagonal precision or a prior mean is
 * PCD_NOT_SUPPORTED, as the generative snapshot refuses them
 * (Network.cs:1334-1338).  Waits for the device. */
int pcd_pc_model_load_record(pcd_model* model, int layer, const void* record, size_t bytes);

/* Model properties (levels, sizes, dtype) for host wrappers. */
int pcd_pc_model_info(const pcd_model* model, int* levels, int* sizes, int max_sizes, int* dtype);

/* Relaxation options (no counterpart in the reference; tuning and profiling
 * hooks for the host wrappers and the benchmark):
 *   use_graph    capture the T-step loop in a hipGraph and replay it (default
 *                1); graphs are cached per call shape (batch, steps, tile, and
 *                for pcd_pc_relax_ragged also requests, exit rule, threshold)
 *   tile, tile_n force a GEMM tile (0 = automatic choice): tile sets rows and
 *                columns, tile_n then the columns; supported 64 x 64,
 *                64 x 128, 64 x 256, 128 x 128, 256 x 128, 256 x 256 and
 *                32 x 32 (the four waves of a workgroup share the tile's K;
 *                the automatic choice for a settling with fewer 64 x 64
 *                error-phase tiles than CUs, unless `persistent` is on)
 *   tile_order   0: every XCD runs an eighth of each problem's tiles (default);
 *                1: every XCD runs one contiguous eighth of the phase's tiles
 *   split_k      1: phases with fewer tiles than half the CUs split K over
 *                several workgroups per tile (default); 0: never
 *   k_stagger    S > 1: GEMM tile (tm, tn) of a settling phase sums its K
 *                stages starting at stage (tm + tn) % S, so tiles sharing
 *                operand rows do not all miss in L2 on the same rows at once;
 *                0 or 1: every tile sums from stage 0; -1: automatic, a
 *                quarter of the longest K sweep's stages, half of them when
 *                the batch fits one row tile (at least 2).  Default
 *                -1 for 16-bit models, 0 for fp32.  With S > 1 a row's bits
 *                depend on where it falls in the batch (they stay the same run
 *                to run); with 0 a row's result is independent of the other
 *                rows.  At most 64.
 *   ragged_tiles 1: before each step of pcd_pc_relax_ragged, list the row tiles
 *                that still hold a running row, and deal only those tiles over
 *                the XCDs (default); 0: launch every tile, and let tiles whose
 *                rows have all finished return at once.  Results are the same.
 *   direct       1: 16-bit batches of at most 64 rows take the direct-weight
 *                tile (weights from a fragment-major copy straight into
 *                registers) where the model keeps that copy, which 16-bit
 *                models with at least one such tile per CU in their error
 *                phase do (default); 0: the 64 x 64 tile; 2: the direct tile
 *                for every 16-bit batch of at most 64 rows (the copy, as much
 *                device memory as W and W^T, is made on first use).  A row's
 *                bits depend on the tile.
 *   nt_store     -1: the settling epilogues' row stores are non-temporal for
 *                16-bit models (default); 0: ordinary stores; 1: non-temporal.
 *                Results are the same.
 *   nt_load      the same for the epilogues' loads of the fp32 states.
 *   ragged_order 1: pcd_pc_relax_ragged settles the requests in decreasing
 *                step budget (rows permuted on the device and back), so rows
 *                that stop early fill whole row tiles that drop out (default);
 *                0: in the caller's order.  fp32 results are the same.
 *   profile      while set, pcd_pc_relax and pcd_pc_relax_ragged run eagerly and
 *                time every phase launch with HIP events (pcd_pc_profile_result)
 *   split_min    fewest K stages a split-K range of a settling phase takes
 *                (0, the default: 4 on the 32 x 32 tile, 12 on the others;
 *                fewer gives more, shorter ranges)
 *   persistent   1: a fixed-step fp32 settling whose phases deal at most two
 *                workgroups per CU (64 x 64 tiles, at most 6 problems a phase)
 *                runs as one cooperative launch of the whole step loop, with
 *                grid barriers between the phases; the call then waits for
 *                the settling.  Results are the phase launches' bit for bit.
 *                Default 0: on MI355X a grid barrier costs about what a graph
 *                node's launch does, and the graph replay is faster.
 *   persist_spin polls of a persistent grid barrier before it gives up (the
 *                call then fails with PCD_HIP_ERROR and every workgroup exits);
 *                default 4194304
 *   persist_grid workgroups of the persistent launch, a multiple of 8 (0:
 *                automatic; capped at what the device holds at once) */
int pcd_pc_set_option(pcd_model* model, const char* name, int value);
/* Average duration (ms) of the error-phase and update-phase kernels over the
 * launches of the last profiled call, and their launch counts. */
int pcd_pc_profile_result(pcd_model* model, float* error_phase_ms, float* update_phase_ms, int* launches);

#ifdef __cplusplus
}
#endif
#endif /* PCDEVICE_H */
