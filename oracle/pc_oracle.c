/*
 * pc_oracle.c -- CPU restatement of the reference's batched predictive-coding
 * relaxation.  TEST INFRASTRUCTURE ONLY: the checker that the HIP library is
 * measured against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path (predicitivecoding_amd)
 * never links, loads or calls it.
 *
 * The reference is C# (.NET 10) and cannot be compiled in this image, so this
 * file restates its equations from the source text:
 *
 *   PredictiveCoding.Device/BatchedPcForward.cs:36-139   batched step loop
 *   PredicitiveCoding/Model/Layer.cs:212-221             ComputePrediction
 *   PredicitiveCoding/Model/Layer.cs:234-258             SetPredictionError
 *   PredicitiveCoding/Model/Layer.cs:273-309             UpdateState
 *   PredicitiveCoding/Model/Layer.cs:437-450             LocalEnergy
 *   PredicitiveCoding/Networks/Network.cs:75-131         InferCore + FFG
 *   PredicitiveCoding/Networks/Network.cs:139-155        Learn
 *   PredicitiveCoding/Networks/Network.cs:253-278        ClassEnergies
 *   PredicitiveCoding/Networks/Network.cs:369-415        PredictCore (min-energy class)
 *   PredicitiveCoding/Model/Layer.cs:320-333             UpdateWeights
 *   PredicitiveCoding/Networks/Network.cs:876-907        SettleAdaptive (exit rule)
 *   PredicitiveCoding/Networks/Network.cs:1080-1093      InferGetTop(resetState)
 *   PredicitiveCoding/Core/Activation.cs:34-132          f and f'
 *   PredictiveCoding.LLM/Model/Layers.cs:42-50           GELU (tanh approximation)
 *   PredictiveCoding.LLM/Autograd/Autograd.cs:303-325    GELU derivative
 *   PredictiveCoding.LLM/Infrastructure/Gemm.cs:32-60    CpuGemmProvider (+ mixed rounding)
 *   PredictiveCoding.LLM/Infrastructure/Gemm.cs:106-124  RowIkj
 *   PredicitiveCoding/Core/TensorUtils.cs:379-401        bf16 round-to-nearest-even
 *
 * Model (s_l = sizes[l], l = 0..L-1; layer 0 is clamped to the input):
 *   W_l  [s_{l-1} x s_l] row-major, b_l [s_{l-1}], scalar precision P_l.
 *   pre_l  = W_l mu_l + b_l,   pred_l = f(pre_l)                 (l = 1..L-1)
 *   e_l    = P_l (mu_l - pred_{l+1})  for l <= L-2,  e_{L-1} = 0 (flat prior)
 *   mu_l  -= eta (e_l - W_l^T [f'(pre_l) . e_{l-1}] + lambda sign(mu_l))
 *   energy = sum_{l=0}^{L-2} 0.5 |e_l|^2 / P_l   (pre-update, as Network.cs:939-945)
 * All layers see the same pre-step snapshot (Jacobi order, Network.cs:91-110).
 *
 * Parity pins for every function here live in tests/test_oracle_*.py (closed
 * forms from the reference's own tests, autograd of the energy, library
 * rounding routines, brute force on tiny nets).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { ACT_LINEAR = 0, ACT_TANH = 1, ACT_RELU = 2, ACT_SIGMOID = 3, ACT_GELU = 4 };
enum { ROUND_NONE = 0, ROUND_F16 = 1, ROUND_BF16 = 2 };
enum { EXIT_NONE = 0, EXIT_RELATIVE = 1, EXIT_ABSOLUTE = 2 };

#define GELU_C 0.7978845608f /* sqrt(2/pi), Layers.cs:43 */
#define GELU_A 0.044715f

/* ---------------------------------------------------------------- activations */

/* f(x): Activation.cs:34-72 (Linear/Tanh/ReLU/Sigmoid), Layers.cs:42-50 (GELU). */
static inline float act_f32(int act, float x) {
    switch (act) {
    case ACT_TANH: return tanhf(x);
    case ACT_RELU: return x > 0.f ? x : 0.f;
    case ACT_SIGMOID: return 1.f / (1.f + expf(-x));
    case ACT_GELU: return 0.5f * x * (1.f + tanhf(GELU_C * (x + GELU_A * x * x * x)));
    default: return x;
    }
}

/* f'(pre) given y = f(pre): Activation.cs:86-132; GELU from pre, Autograd.cs:313-318. */
static inline float dact_f32(int act, float pre, float y) {
    switch (act) {
    case ACT_TANH: return 1.f - y * y;
    case ACT_RELU: return pre > 0.f ? 1.f : 0.f;
    case ACT_SIGMOID: return y * (1.f - y);
    case ACT_GELU: {
        float u = GELU_C * (pre + GELU_A * pre * pre * pre);
        float t = tanhf(u);
        float dudv = GELU_C * (1.f + 3.f * GELU_A * pre * pre);
        return 0.5f * (1.f + t) + 0.5f * pre * (1.f - t * t) * dudv;
    }
    default: return 1.f;
    }
}

static inline double act_f64(int act, double x) {
    const double c = 0.7978845608028654, a = 0.044715;
    switch (act) {
    case ACT_TANH: return tanh(x);
    case ACT_RELU: return x > 0.0 ? x : 0.0;
    case ACT_SIGMOID: return 1.0 / (1.0 + exp(-x));
    case ACT_GELU: return 0.5 * x * (1.0 + tanh(c * (x + a * x * x * x)));
    default: return x;
    }
}

static inline double dact_f64(int act, double pre, double y) {
    const double c = 0.7978845608028654, a = 0.044715;
    switch (act) {
    case ACT_TANH: return 1.0 - y * y;
    case ACT_RELU: return pre > 0.0 ? 1.0 : 0.0;
    case ACT_SIGMOID: return y * (1.0 - y);
    case ACT_GELU: {
        double t = tanh(c * (pre + a * pre * pre * pre));
        return 0.5 * (1.0 + t) + 0.5 * pre * (1.0 - t * t) * c * (1.0 + 3.0 * a * pre * pre);
    }
    default: return 1.0;
    }
}

void pco_act_apply_f32(int act, const float* x, float* y, long n) {
    for (long i = 0; i < n; i++) y[i] = act_f32(act, x[i]);
}
void pco_act_deriv_f32(int act, const float* pre, const float* y, float* d, long n) {
    for (long i = 0; i < n; i++) d[i] = dact_f32(act, pre[i], y[i]);
}
void pco_act_apply_f64(int act, const double* x, double* y, long n) {
    for (long i = 0; i < n; i++) y[i] = act_f64(act, x[i]);
}
void pco_act_deriv_f64(int act, const double* pre, const double* y, double* d, long n) {
    for (long i = 0; i < n; i++) d[i] = dact_f64(act, pre[i], y[i]);
}

/* ------------------------------------------------------------- 16-bit rounding */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 round-to-nearest-even with NaN kept NaN: TensorUtils.cs:386-395. */
static inline uint16_t bf16_bits(float x) {
    uint32_t u = f2u(x);
    if (isnan(x)) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t rounding = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + rounding) >> 16);
}
static inline float bf16_round(float x) { return u2f((uint32_t)bf16_bits(x) << 16); }

/* IEEE binary16 round-to-nearest-even (the rounding System.Half applies when
 * TensorPrimitives.ConvertToHalf runs in Gemm.cs:53-60), widened back to float.
 * Overflow saturates to +-inf; subnormals are rounded on the 2^-24 grid. */
static inline float f16_round(float x) {
    if (isnan(x) || isinf(x)) return x;
    float ax = fabsf(x);
    if (ax >= 65520.f) return copysignf(INFINITY, x); /* rounds past max half 65504 */
    if (ax < 6.103515625e-05f) {                       /* subnormal range: grid 2^-24 */
        float q = rintf(ax * 16777216.f);              /* rint = nearest-even */
        return copysignf(q / 16777216.f, x);
    }
    /* normal: keep 10 mantissa bits of 23, round half to even */
    uint32_t u = f2u(ax);
    uint32_t lsb = (u >> 13) & 1u;
    u += 0x0FFFu + lsb;
    u &= ~0x1FFFu;
    return copysignf(u2f(u), x);
}

static inline float round_op(int mode, float x) {
    return mode == ROUND_BF16 ? bf16_round(x) : mode == ROUND_F16 ? f16_round(x) : x;
}

void pco_round(int mode, const float* x, float* y, long n) {
    for (long i = 0; i < n; i++) y[i] = round_op(mode, x[i]);
}
void pco_bf16_bits(const float* x, uint16_t* bits, long n) {
    for (long i = 0; i < n; i++) bits[i] = bf16_bits(x[i]);
}

/* -------------------------------------------------------------------- GEMM */

/* C[m,n] = A[m,k] B[k,n], row-major, per output row an i-k-j accumulation that
 * skips zero A entries (Gemm.cs:106-124), rows in parallel (Gemm.cs:35).  Rows
 * are processed four at a time so each B row is streamed once per four output
 * rows; every output element still accumulates its k terms in increasing k in
 * float, exactly the per-element order RowIkj uses. */
static void gemm_rowikj(const float* a, int m, int k, const float* b, int n, float* c) {
    memset(c, 0, sizeof(float) * (size_t)m * (size_t)n);
    int nblk = (m + 3) / 4;
#pragma omp parallel for schedule(dynamic, 1)
    for (int blk = 0; blk < nblk; blk++) {
        int i0 = blk * 4, i1 = i0 + 4 < m ? i0 + 4 : m;
        for (int l = 0; l < k; l++) {
            const float* brow = b + (size_t)l * n;
            for (int i = i0; i < i1; i++) {
                float av = a[(size_t)i * k + l];
                if (av == 0.f) continue;
                float* crow = c + (size_t)i * n;
                for (int j = 0; j < n; j++) crow[j] += av * brow[j];
            }
        }
    }
}

/* Gemm.Provider.MatMulMixed semantics (Gemm.cs:44-51): both operands rounded
 * to 16 bits, fp32 accumulation.  b_rounded = 1 states that b already holds
 * rounded values (rounding is idempotent, so skipping it changes nothing). */
static void gemm_mixed(const float* a, int m, int k, const float* b, int n, float* c, int round_mode, int b_rounded) {
    if (round_mode == ROUND_NONE) { gemm_rowikj(a, m, k, b, n, c); return; }
    float* ar = malloc(sizeof(float) * (size_t)m * k);
    pco_round(round_mode, a, ar, (long)m * k);
    if (b_rounded) {
        gemm_rowikj(ar, m, k, b, n, c);
    } else {
        float* br = malloc(sizeof(float) * (size_t)k * n);
        pco_round(round_mode, b, br, (long)k * n);
        gemm_rowikj(ar, m, k, br, n, c);
        free(br);
    }
    free(ar);
}

void pco_gemm(const float* a, int m, int k, const float* b, int n, float* c, int round_mode) {
    gemm_mixed(a, m, k, b, n, c, round_mode, 0);
}

void pco_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
int pco_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* --------------------------------------------------- batched relaxation (fp32) */

typedef struct {
    int levels;
    const int* sizes;
    int act;
    float eta, act_reg;
    int ffg;
    const float* W_all;   /* W_1..W_{L-1} concatenated, W_l is [s_{l-1} x s_l] */
    const float* b_all;   /* b_1..b_{L-1} concatenated */
    const float* prec;    /* [levels] */
    int round_mode;
    int clamp_top;        /* layer L-1 held at its initial state (Network.cs:79-80, Layer.cs:275) */
} model_t;

static const float* w_of(const model_t* md, int l) {
    size_t off = 0;
    for (int j = 1; j < l; j++) off += (size_t)md->sizes[j - 1] * md->sizes[j];
    return md->W_all + off;
}
static const float* b_of(const model_t* md, int l) {
    size_t off = 0;
    for (int j = 1; j < l; j++) off += (size_t)md->sizes[j - 1];
    return md->b_all + off;
}

static float* transpose(const float* w, int rows, int cols) {
    float* t = malloc(sizeof(float) * (size_t)rows * cols);
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) t[(size_t)c * rows + r] = w[(size_t)r * cols + c];
    return t;
}

/*
 * One batch settled together, BatchedPcForward.cs:36-139, extended with the
 * per-sample energy trace and the SettleAdaptive exit test applied to the
 * batch's summed energy (a batch of one sample is exactly Network.cs:876-907).
 *   exit_rule  EXIT_NONE      fixed steps
 *              EXIT_RELATIVE  stop after a step once prev - E < thr * max(prev, 1e-12)
 *                             (never after the first step), Network.cs:901-903
 *              EXIT_ABSOLUTE  stop after a step once E / batch < thr
 * m: [levels] state buffers [batch x s_l], m[0] already holds the input.
 */
static int relax_batch(const model_t* md, float** m, int batch, int steps,
                       int exit_rule, float exit_thr, float* energy_trace /* [steps x batch] or NULL */,
                       float* final_energy /* total over the batch, or NULL */,
                       float** delta_out /* [levels], delta_out[l] [batch x s_{l-1}] of the last step, or NULL */) {
    int L = md->levels;
    const int* s = md->sizes;
    float** wT = calloc((size_t)L, sizeof(float*));
    float** pre = calloc((size_t)L, sizeof(float*));
    float** pred = calloc((size_t)L, sizeof(float*));
    float** e = calloc((size_t)L, sizeof(float*));
    float *delta = NULL, *g = NULL;
    size_t maxw = 0;
    for (int l = 0; l < L; l++) if ((size_t)s[l] > maxw) maxw = (size_t)s[l];
    delta = malloc(sizeof(float) * (size_t)batch * maxw);
    g = malloc(sizeof(float) * (size_t)batch * maxw);
    float** wr = calloc((size_t)L, sizeof(float*));   /* W_l as the mixed GEMM sees it */
    for (int l = 1; l < L; l++) {
        wT[l] = transpose(w_of(md, l), s[l - 1], s[l]);                 /* :62-64 */
        if (md->round_mode != ROUND_NONE) {
            size_t nw = (size_t)s[l - 1] * s[l];
            wr[l] = malloc(sizeof(float) * nw);
            pco_round(md->round_mode, w_of(md, l), wr[l], (long)nw);
            pco_round(md->round_mode, wT[l], wT[l], (long)nw);
        }
        pre[l] = malloc(sizeof(float) * (size_t)batch * s[l - 1]);
        pred[l] = malloc(sizeof(float) * (size_t)batch * s[l - 1]);
    }
    for (int l = 0; l < L - 1; l++) e[l] = malloc(sizeof(float) * (size_t)batch * s[l]);

    /* TopDown(l), :74-80: pre = M[l] W_l^T + b_l ; pred = f(pre). */
#define TOPDOWN(l)                                                                     \
    do {                                                                               \
        int lo_ = s[(l) - 1];                                                          \
        gemm_mixed(m[l], batch, s[l], wT[l], lo_, pre[l], md->round_mode, 1);          \
        const float* bb_ = b_of(md, l);                                                \
        for (int r_ = 0; r_ < batch; r_++)                                             \
            for (int c_ = 0; c_ < lo_; c_++) pre[l][(size_t)r_ * lo_ + c_] += bb_[c_]; \
        pco_act_apply_f32(md->act, pre[l], pred[l], (long)batch * lo_);               \
    } while (0)

    if (md->ffg)                                                          /* :83-88 */
        for (int l = L - 1; l >= 1; l--) {
            TOPDOWN(l);
            if (l > 1) memcpy(m[l - 1], pred[l], sizeof(float) * (size_t)batch * s[l - 1]);
        }

    double previous = INFINITY;
    double energy = 0.0;
    int step = 0;
    while (step < steps) {
        for (int l = L - 1; l >= 1; l--) TOPDOWN(l);                       /* :95-96 */

        double etot = 0.0;
        for (int l = 0; l < L - 1; l++) {                                  /* :100-108 */
            float pi = md->prec[l];
            size_t n = (size_t)batch * s[l];
            for (size_t i = 0; i < n; i++) e[l][i] = pi * (m[l][i] - pred[l + 1][i]);
            /* LocalEnergy, Layer.cs:449: 0.5 |e|^2 / P, per sample */
            for (int r = 0; r < batch; r++) {
                double ss = 0.0;
                const float* er = e[l] + (size_t)r * s[l];
                for (int c = 0; c < s[l]; c++) ss += (double)er[c] * er[c];
                double el = 0.5 * ss / pi;
                etot += el;
                if (energy_trace) energy_trace[(size_t)step * batch + r] += (float)el;
            }
        }

        for (int l = 1; l < L; l++) {                                      /* :110-127 */
            int size = s[l], lower = s[l - 1];
            size_t n = (size_t)batch * lower;
            pco_act_deriv_f32(md->act, pre[l], pred[l], delta, (long)n);
            for (size_t i = 0; i < n; i++) delta[i] *= e[l - 1][i];
            if (delta_out) memcpy(delta_out[l], delta, sizeof(float) * n);
            if (l == L - 1 && md->clamp_top) continue;                     /* Layer.cs:275 */
            gemm_mixed(delta, batch, lower, wr[l] ? wr[l] : w_of(md, l), size, g, md->round_mode, 1);
            float* state = m[l];
            const float* eself = l < L - 1 ? e[l] : NULL;
            size_t ns = (size_t)batch * size;
            for (size_t i = 0; i < ns; i++) {
                float grad = (eself ? eself[i] : 0.f) - g[i];
                if (md->act_reg > 0.f) {
                    float sg = state[i] > 0.f ? 1.f : state[i] < 0.f ? -1.f : 0.f;
                    grad += md->act_reg * sg;
                }
                state[i] -= md->eta * grad;
            }
        }

        step++;
        energy = etot;
        if (exit_rule == EXIT_RELATIVE && exit_thr > 0.f && isfinite(previous) &&
            (float)previous - (float)energy < exit_thr * fmaxf((float)previous, 1e-12f))
            break;
        if (exit_rule == EXIT_ABSOLUTE && energy / batch < exit_thr) break;
        previous = energy;
    }
#undef TOPDOWN
    if (final_energy) *final_energy = (float)energy;
    for (int l = 0; l < L; l++) { free(wT[l]); free(wr[l]); free(pre[l]); free(pred[l]); free(e[l]); }
    free(wT); free(wr); free(pre); free(pred); free(e); free(delta); free(g);
    return step;
}

static void setup_model(model_t* md, const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                        const float* W_all, const float* b_all, const float* prec, int round_mode) {
    md->levels = levels; md->sizes = sizes; md->act = act; md->eta = eta; md->act_reg = act_reg;
    md->ffg = ffg; md->W_all = W_all; md->b_all = b_all; md->prec = prec; md->round_mode = round_mode;
    md->clamp_top = 0;
}

/*
 * InferGetTopBatch (BatchedPcForward.cs:36-139): free layers start at zero,
 * layer 0 holds x0 [batch x s_0].  Outputs:
 *   out_top     [batch x s_{L-1}]
 *   out_states  all layers l = 0..L-1, each [batch x s_l], concatenated (nullable)
 *   out_energy  [steps x batch] per-sample pre-update energy (nullable)
 * Returns 0, or -1 on invalid arguments (mirroring the reference's exceptions).
 */
int pco_batched_relax(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                      const float* W_all, const float* b_all, const float* prec, int round_mode,
                      const float* x0, int batch, int steps,
                      float* out_top, float* out_states, float* out_energy) {
    if (levels < 2 || batch < 1 || steps < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    float** m = calloc((size_t)levels, sizeof(float*));
    for (int l = 0; l < levels; l++) m[l] = calloc((size_t)batch * sizes[l], sizeof(float));
    memcpy(m[0], x0, sizeof(float) * (size_t)batch * sizes[0]);
    if (out_energy) memset(out_energy, 0, sizeof(float) * (size_t)steps * batch);
    relax_batch(&md, m, batch, steps, EXIT_NONE, 0.f, out_energy, NULL, NULL);
    memcpy(out_top, m[levels - 1], sizeof(float) * (size_t)batch * sizes[levels - 1]);
    if (out_states) {
        size_t off = 0;
        for (int l = 0; l < levels; l++) {
            memcpy(out_states + off, m[l], sizeof(float) * (size_t)batch * sizes[l]);
            off += (size_t)batch * sizes[l];
        }
    }
    for (int l = 0; l < levels; l++) free(m[l]);
    free(m);
    return 0;
}

/*
 * Ragged requests: request r owns rows [row_offsets[r], row_offsets[r+1]) of
 * x0_packed and settles for at most steps[r] steps, leaving early by exit_rule
 * applied to the request's summed energy.  Each request is settled on its own
 * (requests never interact), so this is the per-request loop a packed device
 * launch must reproduce.
 *   steps_used [R], final_energy [R] (request energy at its last step),
 *   out_top [rows x s_{L-1}] packed like the input.
 */
int pco_ragged_relax(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                     const float* W_all, const float* b_all, const float* prec, int round_mode,
                     const float* x0_packed, const int* row_offsets, const int* steps, int requests,
                     int exit_rule, float exit_thr, int* steps_used, float* final_energy, float* out_top) {
    if (levels < 2 || requests < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    int s0 = sizes[0], sl = sizes[levels - 1];
    for (int r = 0; r < requests; r++) {
        int r0 = row_offsets[r], nb = row_offsets[r + 1] - r0;
        if (nb < 1 || steps[r] < 1) return -1;
        float** m = calloc((size_t)levels, sizeof(float*));
        for (int l = 0; l < levels; l++) m[l] = calloc((size_t)nb * sizes[l], sizeof(float));
        memcpy(m[0], x0_packed + (size_t)r0 * s0, sizeof(float) * (size_t)nb * s0);
        float fe = 0.f;
        steps_used[r] = relax_batch(&md, m, nb, steps[r], exit_rule, exit_thr, NULL, &fe, NULL);
        final_energy[r] = fe;
        memcpy(out_top + (size_t)r0 * sl, m[levels - 1], sizeof(float) * (size_t)nb * sl);
        for (int l = 0; l < levels; l++) free(m[l]);
        free(m);
    }
    return 0;
}

/*
 * InferCore with both ends clamped (Network.cs:75-111 with clampTop and a
 * label): layer 0 holds x0, layer L-1 holds top [batch x s_{L-1}] and is never
 * updated (Layer.cs:275), the hidden layers start at zero.  This is the
 * settling inside Network.InferEnergy (:234-244), ClassEnergies (:253-278),
 * PredictCore (:369-415) and Learn (:139-155).  Same outputs as
 * pco_batched_relax.
 */
int pco_clamped_relax(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                      const float* W_all, const float* b_all, const float* prec, int round_mode,
                      const float* x0, const float* top, int batch, int steps,
                      float* out_states, float* out_energy) {
    if (levels < 2 || batch < 1 || steps < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    md.clamp_top = 1;
    float** m = calloc((size_t)levels, sizeof(float*));
    for (int l = 0; l < levels; l++) m[l] = calloc((size_t)batch * sizes[l], sizeof(float));
    memcpy(m[0], x0, sizeof(float) * (size_t)batch * sizes[0]);
    memcpy(m[levels - 1], top, sizeof(float) * (size_t)batch * sizes[levels - 1]);
    if (out_energy) memset(out_energy, 0, sizeof(float) * (size_t)steps * batch);
    relax_batch(&md, m, batch, steps, EXIT_NONE, 0.f, out_energy, NULL, NULL);
    if (out_states) {
        size_t off = 0;
        for (int l = 0; l < levels; l++) {
            memcpy(out_states + off, m[l], sizeof(float) * (size_t)batch * sizes[l]);
            off += (size_t)batch * sizes[l];
        }
    }
    for (int l = 0; l < levels; l++) free(m[l]);
    free(m);
    return 0;
}

/*
 * Minimum-energy classification, Network.PredictCore (Network.cs:369-415) and
 * ClassEnergies (:253-278), one sample at a time as the reference runs it:
 * for every class c the hidden states are zeroed, the top is clamped to
 * one-hot(c) and the network settles for `steps` steps; F(x, c) is the energy
 * of the last step's (pre-update) errors (ComputeEnergyCore, :939-945).  The
 * class is the first c with the smallest F (strict <, :395); the winner's
 * energy is F(x, c*) (the reference's re-run of the winner repeats the same
 * deterministic settling).
 *   class_energies [batch x C] (nullable), best_class [batch], best_energy [batch]
 */
int pco_classify(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                 const float* W_all, const float* b_all, const float* prec, int round_mode,
                 const float* x0, int batch, int steps,
                 float* class_energies, int* best_class, float* best_energy) {
    if (levels < 2 || batch < 1 || steps < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    md.clamp_top = 1;
    const int C = sizes[levels - 1], s0 = sizes[0];
    float** m = calloc((size_t)levels, sizeof(float*));
    for (int l = 0; l < levels; l++) m[l] = calloc((size_t)sizes[l], sizeof(float));
    float* fc = malloc(sizeof(float) * (size_t)C);
    for (int b = 0; b < batch; b++) {
        float best = 3.402823466e38f;   /* float.MaxValue, :382 */
        int bc = 0;
        for (int c = 0; c < C; c++) {
            for (int l = 1; l < levels; l++) memset(m[l], 0, sizeof(float) * sizes[l]);
            memcpy(m[0], x0 + (size_t)b * s0, sizeof(float) * s0);
            m[levels - 1][c] = 1.f;
            float fe = 0.f;
            relax_batch(&md, m, 1, steps, EXIT_NONE, 0.f, NULL, &fe, NULL);
            fc[c] = fe;
            if (class_energies) class_energies[(size_t)b * C + c] = fe;
            if (fe < best) { best = fe; bc = c; }
        }
        best_class[b] = bc;
        best_energy[b] = fc[bc];   /* the winner's re-run, :400-406 */
    }
    free(fc);
    for (int l = 0; l < levels; l++) free(m[l]);
    free(m);
    return 0;
}

/*
 * Adaptive minimum-energy classification, Network.PredictAdaptive
 * (Network.cs:803-840) with SettleCandidate (:851-867) and SettleAdaptive
 * (:876-907): every class candidate c of sample b settles from zero hidden
 * states with the top clamped to one-hot(c), for at most max_steps steps,
 * leaving after a step once prev - E < epsilon * max(prev, 1e-12) (never after
 * the first step; epsilon <= 0 never leaves).  F(b, c) is the energy of the
 * candidate's last step; the class is the first c with the smallest F
 * (strictly smaller than float.MaxValue to win, :822); the winner is settled
 * again (:826-828), which repeats its candidate settling exactly, so its
 * steps count twice and its energy is F(b, c*).  Outputs (each nullable):
 *   class_energies [batch x C], class_steps [batch x C], best_class [batch],
 *   best_energy [batch], steps_used [batch] = sum_c steps(b, c) + steps(b, c*).
 */
int pco_classify_adaptive(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
                          const float* W_all, const float* b_all, const float* prec, int round_mode,
                          const float* x0, int batch, int max_steps, float epsilon,
                          float* class_energies, int* class_steps, int* best_class, float* best_energy,
                          int* steps_used) {
    if (levels < 2 || batch < 1 || max_steps < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    md.clamp_top = 1;
    const int C = sizes[levels - 1], s0 = sizes[0];
    float** m = calloc((size_t)levels, sizeof(float*));
    for (int l = 0; l < levels; l++) m[l] = calloc((size_t)sizes[l], sizeof(float));
    float* fc = malloc(sizeof(float) * (size_t)C);
    int* sc = malloc(sizeof(int) * (size_t)C);
    for (int b = 0; b < batch; b++) {
        float best = 3.402823466e38f;   /* float.MaxValue, :814 */
        int bc = 0, total = 0;
        for (int c = 0; c < C; c++) {
            for (int l = 1; l < levels; l++) memset(m[l], 0, sizeof(float) * sizes[l]);
            memcpy(m[0], x0 + (size_t)b * s0, sizeof(float) * s0);
            m[levels - 1][c] = 1.f;
            float fe = 0.f;
            sc[c] = relax_batch(&md, m, 1, max_steps, EXIT_RELATIVE, epsilon, NULL, &fe, NULL);
            fc[c] = fe;
            total += sc[c];
            if (class_energies) class_energies[(size_t)b * C + c] = fe;
            if (class_steps) class_steps[(size_t)b * C + c] = sc[c];
            if (fe < best) { best = fe; bc = c; }
        }
        if (best_class) best_class[b] = bc;
        if (best_energy) best_energy[b] = fc[bc];
        if (steps_used) steps_used[b] = total + sc[bc];
    }
    free(fc);
    free(sc);
    for (int l = 0; l < levels; l++) free(m[l]);
    free(m);
    return 0;
}

/*
 * Learning step, Network.Learn (Network.cs:139-155): settle with input and
 * label clamped, then for every layer l = 1..L-1 Layer.UpdateWeights
 * (Layer.cs:320-333) with the last step's delta_l = f'(pre_l) . e_{l-1}
 * (pre-update) and the settled (post-update) mu_l:
 *   W_l += eta_w delta_l (x) mu_l ;  b_l += eta_w delta_l ;  W_l -= eta_w lambda W_l.
 * A batch of B samples applies the sum of the B per-sample updates, all taken
 * at the weights before the call (B = 1 is exactly Learn).
 * With a 16-bit round_mode the settling runs on rounded operands and the fp32
 * W_all are the master weights, Network.LearnMixed's scheme (Network.cs:158-181);
 * delta is then taken as the settling's W^T GEMM consumed it, rounded to the
 * operand type (the reference's per-sample path keeps it fp32).
 * W_all and b_all are updated in place; out_energy [batch] (nullable) is each
 * sample's energy at the last step (the ComputeEnergy the trainer reads).
 */
int pco_learn(const int* sizes, int levels, int act, float eta, float act_reg, int ffg,
              float* W_all, float* b_all, const float* prec, int round_mode,
              const float* x0, const float* labels, int batch, int steps,
              float eta_w, float weight_decay, float* out_energy,
              const float* hidden_in, float* hidden_out) {
    if (levels < 2 || batch < 1 || steps < 1) return -1;
    model_t md;
    setup_model(&md, sizes, levels, act, eta, act_reg, ffg, W_all, b_all, prec, round_mode);
    md.clamp_top = 1;
    const int L = levels;
    float** m = calloc((size_t)L, sizeof(float*));
    float** d = calloc((size_t)L, sizeof(float*));
    for (int l = 0; l < L; l++) m[l] = calloc((size_t)batch * sizes[l], sizeof(float));
    for (int l = 1; l < L; l++) d[l] = calloc((size_t)batch * sizes[l - 1], sizeof(float));
    memcpy(m[0], x0, sizeof(float) * (size_t)batch * sizes[0]);
    memcpy(m[L - 1], labels, sizeof(float) * (size_t)batch * sizes[L - 1]);
    /* Learn settles from the hidden states the network holds (ReadAllLayers,
     * Network.cs:143, restores each layer's persisted Mu; InferCore resets
     * nothing); hidden_in carries them, null is a network at zero.  The
     * settled hidden states go to hidden_out, the Mu that _store.Write
     * persists for the next call (:150-151). */
    size_t hoff = 0;
    if (hidden_in)
        for (int l = 1; l <= L - 2; l++) {
            memcpy(m[l], hidden_in + hoff, sizeof(float) * (size_t)batch * sizes[l]);
            hoff += (size_t)batch * sizes[l];
        }
    float* trace = calloc((size_t)steps * batch, sizeof(float));
    relax_batch(&md, m, batch, steps, EXIT_NONE, 0.f, trace, NULL, d);
    hoff = 0;
    if (hidden_out)
        for (int l = 1; l <= L - 2; l++) {
            memcpy(hidden_out + hoff, m[l], sizeof(float) * (size_t)batch * sizes[l]);
            hoff += (size_t)batch * sizes[l];
        }
    if (out_energy) memcpy(out_energy, trace + (size_t)(steps - 1) * batch, sizeof(float) * batch);
    free(trace);
    for (int l = 1; l < L; l++) {
        float* W = (float*)w_of(&md, l);
        float* bb = (float*)b_of(&md, l);
        const int lo = sizes[l - 1], sz = sizes[l];
        if (round_mode != ROUND_NONE) pco_round(round_mode, d[l], d[l], (long)batch * lo);
        float* dW = calloc((size_t)lo * sz, sizeof(float));
        float* db = calloc((size_t)lo, sizeof(float));
        for (int r = 0; r < batch; r++) {                   /* OuterProduct(delta, mu), summed */
            const float* dr = d[l] + (size_t)r * lo;
            const float* mr = m[l] + (size_t)r * sz;
            for (int i = 0; i < lo; i++) {
                db[i] += dr[i];
                for (int j = 0; j < sz; j++) dW[(size_t)i * sz + j] += dr[i] * mr[j];
            }
        }
        const size_t nw = (size_t)lo * sz;
        for (size_t k = 0; k < nw; k++) W[k] += eta_w * dW[k];
        for (int i = 0; i < lo; i++) bb[i] += eta_w * db[i];
        if (weight_decay > 0.f)
            for (size_t k = 0; k < nw; k++) W[k] += (-eta_w * weight_decay) * W[k];
        free(dW);
        free(db);
    }
    for (int l = 0; l < L; l++) { free(m[l]); free(d[l]); }
    free(m);
    free(d);
    return 0;
}

/* ------------------------------------------- per-sample relaxation (fp64) */

/*
 * Network.InferGetTop(x, steps, resetState: true) for one sample at a time in
 * double precision: Layer.ComputePrediction (MatVec W mu + b, f), then
 * SetPredictionError for every layer, then UpdateState for every free layer
 * (Network.cs:91-110).  The matrix-vector products are plain dot products,
 * the structure of TensorUtils.MatVecMul / MatVecMulT rather than a GEMM, so
 * agreement with pco_batched_relax also checks the batched reshaping.
 * Same output layout as pco_batched_relax; energies per sample per step.
 */
int pco_persample_relax_f64(const int* sizes, int levels, int act, double eta, double act_reg, int ffg,
                            const double* W_all, const double* b_all, const double* prec,
                            const double* x0, const double* top /* [batch x s_{L-1}] clamped top, or NULL */,
                            int batch, int steps,
                            double* out_top, double* out_states, double* out_energy) {
    if (levels < 2 || batch < 1 || steps < 1) return -1;
    int L = levels;
    size_t* woff = calloc((size_t)L, sizeof(size_t));
    size_t* boff = calloc((size_t)L, sizeof(size_t));
    for (int l = 2; l < L; l++) {
        woff[l] = woff[l - 1] + (size_t)sizes[l - 2] * sizes[l - 1];
        boff[l] = boff[l - 1] + (size_t)sizes[l - 2];
    }
    double** mu = calloc((size_t)L, sizeof(double*));
    double** pre = calloc((size_t)L, sizeof(double*));
    double** pred = calloc((size_t)L, sizeof(double*));
    double** e = calloc((size_t)L, sizeof(double*));
    for (int l = 0; l < L; l++) {
        mu[l] = calloc((size_t)sizes[l], sizeof(double));
        e[l] = calloc((size_t)sizes[l], sizeof(double));
        if (l >= 1) {
            pre[l] = calloc((size_t)sizes[l - 1], sizeof(double));
            pred[l] = calloc((size_t)sizes[l - 1], sizeof(double));
        }
    }
    for (int smp = 0; smp < batch; smp++) {
        for (int l = 1; l < L; l++) memset(mu[l], 0, sizeof(double) * sizes[l]);   /* resetState */
        memcpy(mu[0], x0 + (size_t)smp * sizes[0], sizeof(double) * sizes[0]);    /* ClampLayer(0) */
        if (top) memcpy(mu[L - 1], top + (size_t)smp * sizes[L - 1], sizeof(double) * sizes[L - 1]);

#define PREDICT(l)                                                                       \
        do {                                                                             \
            const double* W_ = W_all + woff[l];                                          \
            const double* b_ = b_all + boff[l];                                          \
            int lo_ = sizes[(l) - 1], sz_ = sizes[l];                                    \
            for (int r_ = 0; r_ < lo_; r_++) {                                           \
                double acc_ = 0.0;                                                       \
                for (int c_ = 0; c_ < sz_; c_++) acc_ += W_[(size_t)r_ * sz_ + c_] * mu[l][c_]; \
                pre[l][r_] = acc_ + b_[r_];                                              \
                pred[l][r_] = act_f64(act, pre[l][r_]);                                  \
            }                                                                            \
        } while (0)

        if (ffg)                                                           /* Network.cs:121-131 */
            for (int l = L - 1; l >= 1; l--) {
                PREDICT(l);
                if (l > 1) memcpy(mu[l - 1], pred[l], sizeof(double) * sizes[l - 1]);
            }

        for (int step = 0; step < steps; step++) {
            for (int l = L - 1; l >= 1; l--) PREDICT(l);
            double etot = 0.0;
            for (int l = 0; l < L - 1; l++) {
                double ss = 0.0;
                for (int i = 0; i < sizes[l]; i++) {
                    e[l][i] = prec[l] * (mu[l][i] - pred[l + 1][i]);
                    ss += e[l][i] * e[l][i];
                }
                etot += 0.5 * ss / prec[l];
            }
            memset(e[L - 1], 0, sizeof(double) * sizes[L - 1]);
            if (out_energy) out_energy[(size_t)step * batch + smp] = etot;
            for (int l = 1; l < L; l++) {                                  /* UpdateState */
                if (l == L - 1 && top) continue;                           /* clamped top, Layer.cs:275 */
                const double* W_ = W_all + woff[l];
                int lo = sizes[l - 1], sz = sizes[l];
                double* grad = calloc((size_t)sz, sizeof(double));
                for (int r = 0; r < lo; r++) {                             /* MatVecMulT */
                    double d = dact_f64(act, pre[l][r], pred[l][r]) * e[l - 1][r];
                    for (int c = 0; c < sz; c++) grad[c] += W_[(size_t)r * sz + c] * d;
                }
                for (int c = 0; c < sz; c++) {
                    double gr = e[l][c] - grad[c];
                    if (act_reg > 0.0) gr += act_reg * (mu[l][c] > 0 ? 1.0 : mu[l][c] < 0 ? -1.0 : 0.0);
                    mu[l][c] -= eta * gr;
                }
                free(grad);
            }
        }
#undef PREDICT
        memcpy(out_top + (size_t)smp * sizes[L - 1], mu[L - 1], sizeof(double) * sizes[L - 1]);
        if (out_states) {
            size_t off = 0;
            for (int l = 0; l < L; l++) {
                memcpy(out_states + off + (size_t)smp * sizes[l], mu[l], sizeof(double) * sizes[l]);
                off += (size_t)batch * sizes[l];
            }
        }
    }
    for (int l = 0; l < L; l++) { free(mu[l]); free(e[l]); free(pre[l]); free(pred[l]); }
    free(mu); free(pre); free(pred); free(e); free(woff); free(boff);
    return 0;
}
