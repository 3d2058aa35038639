/*
 * decode_gemv.c -- calling librlxq from plain C, the way a non-Python host
 * (a Rust or C++ runtime) does: one Q4_1 decode GEMV, y = x . W^T with
 * W [N, K] in GGUF Q4_1 blocks, checked against a double-precision loop.
 *
 * Exit status: 0 ok, 1 wrong result or failed call, 77 no gfx950 device.
 * Build (build.py does this): gcc -std=c99 -O2 -D__HIP_PLATFORM_AMD__
 *   -I include -I /opt/rocm/include decode_gemv.c -L lib -lrlxq -lamdhip64
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "rlxq.h"

enum { N = 768, K = 2048, BLK = 20 };

static uint32_t rng = 12345u;
static uint32_t next(void) { rng = rng * 1664525u + 1013904223u; return rng >> 8; }

/* IEEE half to double (normal numbers and zero are all this example makes) */
static double half_to_double(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    const double v = e ? ldexp(1.0 + m / 1024.0, e - 15) : ldexp(m / 1024.0, -14);
    return s ? -v : v;
}

int main(void) {
    rlxq_ctx* ctx = NULL;
    int rc = rlxq_init(0, &ctx);
    if (rc != RLXQ_OK) {
        printf("decode_gemv: no usable device (%s)\n", rlxq_strerror(rc));
        return 77;
    }
    const size_t wbytes = (size_t)N * (K / 32) * BLK;
    uint8_t* w = malloc(wbytes);
    float* x = malloc(sizeof(float) * K);
    float* y = malloc(sizeof(float) * N);
    double* want = malloc(sizeof(double) * N);
    if (!w || !x || !y || !want) return 1;
    /* GGUF block_q4_1: f16 d, f16 m, 16 bytes of nibbles (byte j: element j
     * in the low nibble, element j + 16 in the high one); w = d * q + m */
    for (size_t b = 0; b < (size_t)N * (K / 32); b++) {
        uint8_t* p = w + b * BLK;
        const uint16_t d = (uint16_t)(0x2000u | (next() & 0x3ffu)); /* 2^-7 .. 2^-6 */
        const uint16_t m = (uint16_t)(0xb000u | (next() & 0x3ffu)); /* -(2^-3 .. 2^-2) */
        p[0] = (uint8_t)d; p[1] = (uint8_t)(d >> 8);
        p[2] = (uint8_t)m; p[3] = (uint8_t)(m >> 8);
        for (int j = 0; j < 16; j++) p[4 + j] = (uint8_t)next();
    }
    for (int k = 0; k < K; k++) x[k] = (float)((int)(next() % 2001) - 1000) / 500.0f;
    for (int n = 0; n < N; n++) {
        double acc = 0.0;
        for (int b = 0; b < K / 32; b++) {
            const uint8_t* p = w + ((size_t)n * (K / 32) + b) * BLK;
            const double d = half_to_double((uint16_t)(p[0] | p[1] << 8));
            const double m = half_to_double((uint16_t)(p[2] | p[3] << 8));
            for (int e = 0; e < 32; e++) {
                const int q = e < 16 ? (p[4 + e] & 15) : (p[4 + e - 16] >> 4);
                acc += (d * q + m) * x[b * 32 + e];
            }
        }
        want[n] = acc;
    }

    void *dx = NULL, *dw = NULL, *dy = NULL;
    if (hipMalloc(&dx, sizeof(float) * K) != hipSuccess || hipMalloc(&dw, wbytes) != hipSuccess ||
        hipMalloc(&dy, sizeof(float) * N) != hipSuccess)
        return 1;
    if (hipMemcpy(dx, x, sizeof(float) * K, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dw, w, wbytes, hipMemcpyHostToDevice) != hipSuccess)
        return 1;
    rc = rlxq_dequant_matmul(ctx, RLXQ_GGUF_Q4_1, 32, dx, RLXQ_F32, dw, NULL, NULL, RLXQ_F32, 1, K, N, dy,
                             RLXQ_F32, NULL);
    if (rc != RLXQ_OK) {
        printf("decode_gemv: %s: %s\n", rlxq_strerror(rc), rlxq_last_error(ctx));
        return 1;
    }
    if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(y, dy, sizeof(float) * N, hipMemcpyDeviceToHost) != hipSuccess)
        return 1;
    double err = 0.0, ref = 0.0;
    for (int n = 0; n < N; n++) {
        err = fmax(err, fabs(y[n] - want[n]));
        ref = fmax(ref, fabs(want[n]));
    }
    printf("decode_gemv: %s, N=%d K=%d, max|y - ref| / max|ref| = %.3g\n", rlxq_last_kernel(ctx), N, K, err / ref);
    (void)hipFree(dx); (void)hipFree(dw); (void)hipFree(dy);
    rlxq_destroy(ctx);
    free(w); free(x); free(y); free(want);
    return err / ref <= 1e-3 ? 0 : 1;
}
