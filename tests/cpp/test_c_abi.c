/* A C translation unit that includes include/rt_hip.h, links librt_hip.so and
 * calls it the way a C or C++ caller of the reference path would (through
 * the declarations a reference-side binding uses).  "cpu": argument checking and
 * size queries, no device needed.  "gpu": the host drop-in with its weight
 * cache, a weight handle, and a captured graph, each checked against the
 * CPU oracle (oracle/liboracle.so: the restatement of the reference's
 * arithmetic; test infrastructure). */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rt_hip.h"
#include "rt_oracle.h"

static int failures = 0;
#define CHECK(c)                                                                  \
    do {                                                                          \
        if (!(c)) {                                                               \
            fprintf(stderr, "FAILED %s:%d: %s (%s)\n", __FILE__, __LINE__, #c,    \
                    rt_hip_last_error());                                         \
            ++failures;                                                           \
        }                                                                         \
    } while (0)

static double normwise(const float* y, const float* ref, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double)y[i] - (double)ref[i]), r = fabs((double)ref[i]);
        if (d > num) num = d;
        if (r > den) den = r;
    }
    return num / (den > 1e-30 ? den : 1e-30);
}

static int cpu_checks(void) {
    CHECK(strstr(rt_hip_version(), "gfx950") != NULL);
    CHECK(rt_hip_gemv_q4k(NULL, NULL, NULL, 16, 256, 1, NULL) == RT_HIP_E_ARG);
    CHECK(strlen(rt_hip_last_error()) > 0);
    CHECK(rt_hip_q4k_tiled_bytes(16, 256) == 2304);
    CHECK(rt_hip_q4k_tiled_bytes(16, 100) == -1);
    CHECK(rt_hip_q4mat_bytes(4, 64) == 256 + 4 * 64 / 32 * 4);
    CHECK(rt_hip_q4mat_scales_offset(4, 64) == 256);
    CHECK(rt_hip_q4mat_bytes(4, 33) == -1);
    {
        char host[64];
        rt_hip_weight* w = NULL;
        CHECK(rt_hip_weight_upload(RT_HIP_Q4K, host, 100, 1, 256, 0, &w) == RT_HIP_E_SHAPE && w == NULL);
        CHECK(rt_hip_weight_upload(99, host, 64, 1, 256, 0, &w) == RT_HIP_E_SHAPE);
        CHECK(rt_hip_host_matmul(RT_HIP_Q4MAT, host, 64, NULL, 1, 128, (const float*)host, (float*)host, 1) ==
              RT_HIP_E_ARG);
    }
    CHECK(rt_hip_graph_launch(NULL, NULL) == RT_HIP_E_ARG);
    CHECK(rt_hip_graph_end(NULL, NULL) == RT_HIP_E_ARG);
    CHECK(rt_hip_weight_free(NULL) == RT_HIP_OK);
    return failures;
}

static void fill(float* v, size_t n, unsigned seed, float scale) {
    /* uniform in [-scale, scale), a plain LCG */
    unsigned s = seed * 2654435761u + 1u;
    for (size_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        v[i] = scale * ((float)(s >> 8) / 8388608.0f - 1.0f);
    }
}

static int gpu_checks(void) {
    const size_t n = 512, k = 1024, nb = n * (k / 256) * 144;
    float* w = malloc(n * k * 4);
    float* x = malloc(64 * k * 4);
    float* y = malloc(64 * n * 4);
    float* ref = malloc(64 * n * 4);
    uint8_t* blocks = malloc(nb);
    fill(w, n * k, 1, 0.05f);
    fill(x, 64 * k, 2, 1.0f);
    CHECK(rt_hip_init(0) == RT_HIP_OK);

    /* host drop-in, Q4_K, M = 1: metal_gemv_q4k_t */
    orc_q4k_quantize(w, n, k, blocks, 1);
    orc_q4k_matmul_t(blocks, n, k, x, 1, ref, 1, 0, n);
    CHECK(rt_hip_host_matmul(RT_HIP_Q4K, blocks, (int64_t)nb, NULL, n, k, x, y, 1) == RT_HIP_OK);
    CHECK(normwise(y, ref, n) <= 1e-5);
    CHECK(rt_hip_host_cache_bytes() == (int64_t)nb);
    {   /* second call: served from the cache, same bits */
        float* y2 = malloc(n * 4);
        CHECK(rt_hip_host_matmul(RT_HIP_Q4K, blocks, (int64_t)nb, NULL, n, k, x, y2, 1) == RT_HIP_OK);
        CHECK(memcmp(y, y2, n * 4) == 0);
        CHECK(rt_hip_host_cache_bytes() == (int64_t)nb);
        free(y2);
    }

    /* host drop-in, Q4Mat, M = 1 and 64: metal_matmul_q4_t */
    {
        uint8_t* packed = malloc(n * k / 2);
        float* scales = malloc(n * k / 32 * 4);
        orc_q4mat_quantize(w, n * k, packed, scales);
        const size_t ms[2] = {1, 64};
        for (int i = 0; i < 2; ++i) {
            orc_q4mat_matmul_t(packed, scales, n, k, x, ms[i], ref);
            CHECK(rt_hip_host_matmul(RT_HIP_Q4MAT, packed, (int64_t)(n * k / 2), scales, n, k, x, y,
                                     (int64_t)ms[i]) == RT_HIP_OK);
            double e = 0.0;
            for (size_t r = 0; r < ms[i]; ++r) {
                const double er = normwise(y + r * n, ref + r * n, n);
                if (er > e) e = er;
            }
            /* M = 1: the GEMV bar; M = 64: bf16 GEMM, operand rounding */
            CHECK(e <= (ms[i] == 1 ? 1e-5 : 2e-2));
        }
        free(packed);
        free(scales);
    }
    CHECK(rt_hip_host_cache_clear() == RT_HIP_OK && rt_hip_host_cache_bytes() == 0);

    /* weight handle (tiled) on device activations, then a captured graph */
    {
        rt_hip_weight* h = NULL;
        float *dx = NULL, *dy = NULL;
        hipStream_t s = NULL;
        CHECK(rt_hip_weight_upload(RT_HIP_Q4K, blocks, (int64_t)nb, n, k, RT_HIP_WEIGHT_TILED, &h) == RT_HIP_OK);
        CHECK(hipMalloc((void**)&dx, k * 4) == hipSuccess && hipMalloc((void**)&dy, n * 4) == hipSuccess);
        CHECK(hipStreamCreate(&s) == hipSuccess);
        CHECK(hipMemcpy(dx, x, k * 4, hipMemcpyHostToDevice) == hipSuccess);
        orc_q4k_matmul_t(blocks, n, k, x, 1, ref, 1, 0, n);
        CHECK(rt_hip_weight_linear(h, dx, NULL, dy, 1, s) == RT_HIP_OK);
        CHECK(hipStreamSynchronize(s) == hipSuccess);
        CHECK(hipMemcpy(y, dy, n * 4, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(normwise(y, ref, n) <= 1e-5);

        rt_hip_graph* g = NULL;
        CHECK(rt_hip_graph_begin(s) == RT_HIP_OK);
        CHECK(rt_hip_weight_linear(h, dx, NULL, dy, 1, s) == RT_HIP_OK);
        CHECK(rt_hip_graph_end(s, &g) == RT_HIP_OK && g != NULL);
        for (int rep = 0; rep < 3; ++rep) {
            CHECK(hipMemset(dy, 0, n * 4) == hipSuccess);
            CHECK(hipDeviceSynchronize() == hipSuccess);
            CHECK(rt_hip_graph_launch(g, s) == RT_HIP_OK);
            CHECK(hipStreamSynchronize(s) == hipSuccess);
            CHECK(hipMemcpy(y, dy, n * 4, hipMemcpyDeviceToHost) == hipSuccess);
            CHECK(normwise(y, ref, n) <= 1e-5);
        }
        CHECK(rt_hip_graph_destroy(g) == RT_HIP_OK);
        CHECK(rt_hip_weight_free(h) == RT_HIP_OK);
        (void)hipFree(dx);
        (void)hipFree(dy);
        (void)hipStreamDestroy(s);
    }
    free(w);
    free(x);
    free(y);
    free(ref);
    free(blocks);
    return failures;
}

int main(int argc, char** argv) {
    const int gpu = argc > 1 && strcmp(argv[1], "gpu") == 0;
    cpu_checks();
    if (gpu) gpu_checks();
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("c abi (%s): all checks passed\n", gpu ? "cpu + gpu" : "cpu");
    return 0;
}
