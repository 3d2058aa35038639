/* Kernel argument block of the dequant-GEMV kernels, shared by the host
 * (g++) and device (hipcc) compilers: plain C types only, so both lay it out
 * identically.  Passed by value as the kernels' single argument. */
#ifndef RLXQ_GEMV_ARGS_H
#define RLXQ_GEMV_ARGS_H
#include <stdint.h>

typedef struct rlxq_gemv_args {
  const void* x;           /* [M, K] activations (f32 or bf16)                 */
  const uint8_t* w;        /* packed weight rows, row stride rb bytes         */
  const void* scales;      /* MLX: [N, K/group] (f32 or bf16), else NULL      */
  const void* biases;      /* MLX: [N, K/group], else NULL                    */
  void* y;                 /* output rows, leading dimension y_ld             */
  const int32_t* row_map;  /* optional: output row of activation row m        */
  const float* row_scale;  /* optional: factor applied to activation row m    */
  int64_t M, N, rb, y_ld;
  int32_t K, group, sb_bf16, y_bf16;
} rlxq_gemv_args;

#endif
