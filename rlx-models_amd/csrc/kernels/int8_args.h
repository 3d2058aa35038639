/* Argument blocks of the int8 kernels (W8A8 GEMM, Int8Block matmul), shared
 * by the host (g++) and device (hipcc) compilers: plain C types only. */
#ifndef RLXQ_INT8_ARGS_H
#define RLXQ_INT8_ARGS_H
#include <stdint.h>

typedef struct rlxq_w8a8_args {
  const int8_t* qx;       /* [M, K] int8 activations (per-row quantised)  */
  const float* sx;        /* [M] activation scales                        */
  const int8_t* wq;       /* [K, N] int8 weights, row-major               */
  const float* sw;        /* [N] weight scales                            */
  void* y;                /* [M, N] output, leading dimension y_ld        */
  int64_t M, N, K, y_ld;
  int32_t tiles_m, tiles_n, y_bf16, pad;
} rlxq_w8a8_args;

typedef struct rlxq_i8b_args {
  const void* x;          /* [M, K] activations, f32 or bf16              */
  const int8_t* wq;       /* [K, N] int8 weights, row-major               */
  const float* scale;     /* [N]                                          */
  const float* zp;        /* [N] zero points, or NULL                     */
  const float* xsum;      /* [M] row sums of x (when zp != NULL)          */
  float* part;            /* [splits, M, N] partial sums (splits > 1)     */
  void* y;                /* [M, N] output (splits == 1)                  */
  int64_t M, N, K, y_ld;
  int32_t kslice;         /* K rows per split (multiple of 128)           */
  int32_t splits, tiles_n, x_bf16, y_bf16, pad;
} rlxq_i8b_args;

#endif
