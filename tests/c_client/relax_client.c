/*
 * A plain C99 caller of libpcdevice_hip.so: only include/pcdevice.h, the way
 * the reference's P/Invoke layer binds the library (no Python, no C++).  It
 * settles a small network through pcd_pc_relax, pcd_pc_relax_noalloc and
 * pcd_pc_relax_ragged in fp32 and bf16, checks an argument error and its
 * message, and compares every result with the CPU oracle (oracle/pc_oracle.c,
 * linked as test infrastructure): |a - b| <= tol (1 + |b|) with tol 1e-4 for
 * fp32 and 2e-3 for bf16 operands against the same-rounding oracle.
 * Exit status 0 when every check holds.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pcdevice.h"

/* oracle entry points (oracle/pc_oracle.c) */
int pco_batched_relax(const int* sizes, int levels, int act, float eta, float act_reg, int ffg, const float* W_all,
                      const float* b_all, const float* prec, int round_mode, const float* x0, int batch, int steps,
                      float* out_top, float* out_states, float* out_energy);
int pco_ragged_relax(const int* sizes, int levels, int act, float eta, float act_reg, int ffg, const float* W_all,
                     const float* b_all, const float* prec, int round_mode, const float* x0_packed,
                     const int* row_offsets, const int* steps, int requests, int exit_rule, float exit_thr,
                     int* steps_used, float* final_energy, float* out_top);
enum { ORACLE_ROUND_NONE = 0, ORACLE_ROUND_BF16 = 2 };

#define LEVELS 4
static const int kSizes[LEVELS] = {20, 48, 33, 6};
static int g_failures = 0;

#define CHECK(call)                                                                       \
    do {                                                                                  \
        int st_ = (call);                                                                 \
        if (st_ != PCD_SUCCESS) {                                                         \
            char msg_[256];                                                               \
            pcd_last_error(msg_, sizeof msg_);                                            \
            printf("FAIL %s:%d: %s -> %d (%s)\n", __FILE__, __LINE__, #call, st_, msg_); \
            exit(1);                                                                      \
        }                                                                                 \
    } while (0)

static unsigned g_seed = 12345u;
static float uniform_pm(float scale) {
    g_seed = g_seed * 1664525u + 1013904223u;
    return ((float)(g_seed >> 8) / 16777216.0f * 2.0f - 1.0f) * scale;
}

static double max_rel(const float* a, const float* b, size_t n) {
    double worst = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double)a[i] - (double)b[i]) / (1.0 + fabs((double)b[i]));
        if (d > worst || d != d) worst = d != d ? INFINITY : d;
    }
    return worst;
}

static void expect(const char* what, double err, double tol) {
    printf("%-40s max rel err %.3e (bound %.0e)%s\n", what, err, tol, err < tol ? "" : "  FAIL");
    if (!(err < tol)) ++g_failures;
}

static void* dev_alloc(size_t bytes) {
    void* p = NULL;
    CHECK(pcd_malloc_async(&p, bytes, NULL));
    return p;
}

int main(void) {
    int version = 0, count = 0;
    CHECK(pcd_version(&version));
    if (pcd_get_device_count(&count) != PCD_SUCCESS || count < 1) {
        printf("FAIL: no device (count %d)\n", count);
        return 1;
    }
    CHECK(pcd_set_device(0));
    printf("libpcdevice_hip %d, %d device(s)\n", version, count);

    /* network: W_l [s_{l-1} x s_l] row-major, b_l [s_{l-1}], concatenated for the oracle */
    size_t wn = 0, bn = 0;
    for (int l = 1; l < LEVELS; ++l) {
        wn += (size_t)kSizes[l - 1] * kSizes[l];
        bn += (size_t)kSizes[l - 1];
    }
    float* W_all = malloc(wn * sizeof(float));
    float* b_all = malloc(bn * sizeof(float));
    const float* W[LEVELS - 1];
    const float* b[LEVELS - 1];
    float prec[LEVELS] = {1.0f, 0.8f, 1.2f, 1.0f};
    {
        size_t wo = 0, bo = 0;
        for (int l = 1; l < LEVELS; ++l) {
            const float scale = sqrtf(3.0f / (float)kSizes[l]);
            W[l - 1] = W_all + wo;
            b[l - 1] = b_all + bo;
            for (int i = 0; i < kSizes[l - 1] * kSizes[l]; ++i) W_all[wo + i] = uniform_pm(scale);
            for (int i = 0; i < kSizes[l - 1]; ++i) b_all[bo + i] = uniform_pm(0.1f);
            wo += (size_t)kSizes[l - 1] * kSizes[l];
            bo += (size_t)kSizes[l - 1];
        }
    }
    const int B = 9, T = 7, s0 = kSizes[0], st = kSizes[LEVELS - 1];
    const float eta = 0.1f;
    float* x = malloc((size_t)B * s0 * sizeof(float));
    for (int i = 0; i < B * s0; ++i) x[i] = uniform_pm(1.0f);

    float* d_x = dev_alloc((size_t)B * s0 * sizeof(float));
    float* d_top = dev_alloc((size_t)B * st * sizeof(float));
    float* d_top2 = dev_alloc((size_t)B * st * sizeof(float));
    float* d_energy = dev_alloc((size_t)T * B * sizeof(float));
    CHECK(pcd_memcpy(d_x, x, (size_t)B * s0 * sizeof(float), PCD_HOST_TO_DEVICE));

    float* top = malloc((size_t)B * st * sizeof(float));
    float* top2 = malloc((size_t)B * st * sizeof(float));
    float* energy = malloc((size_t)T * B * sizeof(float));
    float* rtop = malloc((size_t)B * st * sizeof(float));
    float* renergy = malloc((size_t)T * B * sizeof(float));

    const int dtypes[2] = {PCD_F32, PCD_BF16};
    const int rounds[2] = {ORACLE_ROUND_NONE, ORACLE_ROUND_BF16};
    const double tols[2] = {1e-4, 2e-3};
    for (int k = 0; k < 2; ++k) {
        const char* name = k == 0 ? "fp32" : "bf16";
        char label[64];
        pcd_model* m = NULL;
        CHECK(pcd_pc_model_create(kSizes, LEVELS, PCD_ACT_TANH, eta, 0.0f, 0, W, b, prec, dtypes[k], &m));

        CHECK(pcd_pc_relax(m, d_x, B, T, d_top, NULL, d_energy, NULL));
        CHECK(pcd_device_synchronize());
        CHECK(pcd_memcpy(top, d_top, (size_t)B * st * sizeof(float), PCD_DEVICE_TO_HOST));
        CHECK(pcd_memcpy(energy, d_energy, (size_t)T * B * sizeof(float), PCD_DEVICE_TO_HOST));
        if (pco_batched_relax(kSizes, LEVELS, PCD_ACT_TANH, eta, 0.0f, 0, W_all, b_all, prec, rounds[k], x, B, T,
                              rtop, NULL, renergy) != 0) {
            printf("FAIL: oracle rejected the case\n");
            return 1;
        }
        snprintf(label, sizeof label, "pcd_pc_relax %s top", name);
        expect(label, max_rel(top, rtop, (size_t)B * st), tols[k]);
        snprintf(label, sizeof label, "pcd_pc_relax %s energy", name);
        expect(label, max_rel(energy, renergy, (size_t)T * B), tols[k]);

        /* the allocation-free entry point gives the same bits */
        CHECK(pcd_pc_relax_noalloc(m, d_x, B, T, d_top2, NULL, NULL, NULL));
        CHECK(pcd_device_synchronize());
        CHECK(pcd_memcpy(top2, d_top2, (size_t)B * st * sizeof(float), PCD_DEVICE_TO_HOST));
        printf("%-40s %s\n", "pcd_pc_relax_noalloc == pcd_pc_relax",
               memcmp(top, top2, (size_t)B * st * sizeof(float)) == 0 ? "bit for bit" : "DIFFERS  FAIL");
        if (memcmp(top, top2, (size_t)B * st * sizeof(float)) != 0) ++g_failures;

        /* ragged requests with the reference's relative exit */
        const int offs[4] = {0, 2, 3, 9};
        const int steps[3] = {12, 3, 20};
        int used[3], rused[3];
        float fe[3], rfe[3];
        CHECK(pcd_pc_relax_ragged(m, d_x, offs, steps, 3, PCD_EXIT_RELATIVE, 0.05f, used, d_top, fe, NULL));
        CHECK(pcd_memcpy(top, d_top, (size_t)B * st * sizeof(float), PCD_DEVICE_TO_HOST));
        pco_ragged_relax(kSizes, LEVELS, PCD_ACT_TANH, eta, 0.0f, 0, W_all, b_all, prec, rounds[k], x, offs, steps, 3,
                         PCD_EXIT_RELATIVE, 0.05f, rused, rfe, rtop);
        printf("%-40s device %d %d %d, oracle %d %d %d\n", "pcd_pc_relax_ragged steps used", used[0], used[1],
               used[2], rused[0], rused[1], rused[2]);
        if (k == 0 && (used[0] != rused[0] || used[1] != rused[1] || used[2] != rused[2])) ++g_failures;
        if (k == 0) {
            snprintf(label, sizeof label, "pcd_pc_relax_ragged %s top", name);
            expect(label, max_rel(top, rtop, (size_t)B * st), tols[k]);
            snprintf(label, sizeof label, "pcd_pc_relax_ragged %s energy", name);
            expect(label, max_rel(fe, rfe, 3), tols[k]);
        }

        /* an argument error comes back as a status and a message */
        char msg[256] = {0};
        const int bad = pcd_pc_relax(m, d_x, 0, T, d_top, NULL, NULL, NULL);
        pcd_last_error(msg, sizeof msg);
        printf("%-40s status %d, \"%s\"\n", "pcd_pc_relax with batch 0", bad, msg);
        if (bad != PCD_INVALID_VALUE || strstr(msg, "Empty batch.") == NULL) ++g_failures;

        CHECK(pcd_pc_model_destroy(m));
    }

    CHECK(pcd_free_async(d_x, NULL));
    CHECK(pcd_free_async(d_top, NULL));
    CHECK(pcd_free_async(d_top2, NULL));
    CHECK(pcd_free_async(d_energy, NULL));
    CHECK(pcd_device_synchronize());
    free(W_all);
    free(b_all);
    free(x);
    free(top);
    free(top2);
    free(energy);
    free(rtop);
    free(renergy);
    printf("c-client: %s\n", g_failures ? "FAILED" : "OK");
    return g_failures ? 1 : 0;
}
