/* Kernel argument block of the prefill dequant-GEMM kernels, shared by the
 * host (g++) and device (hipcc) compilers: plain C types only. */
#ifndef RLXQ_GEMM_ARGS_H
#define RLXQ_GEMM_ARGS_H
#include <stdint.h>

typedef struct rlxq_gemm_args {
  const void* x;          /* [M, K] bf16 activations; f16 kernels: the f16
                             rows prepared by rlxq_x16_prep (scaled by a
                             power of two, in the code-unpacking order)    */
  const float* inv_s;     /* f16 kernels: [M] factors undoing the scaling */
  const uint8_t* w;       /* packed weight rows, row stride rb bytes      */
  const void* scales;     /* MLX: [N, K/group] (f32 or bf16), else NULL   */
  const void* biases;     /* MLX: [N, K/group], else NULL                 */
  void* y;                /* [M, N] output, leading dimension y_ld        */
  int64_t M, N, K, rb, y_ld;
  int32_t group, sb_bf16, y_bf16;
  /* f16 kernels: M counts x16 rows prepared in hi/lo pairs (row 2r + 1 the
   * remainder of row 2r); the epilogue adds each pair into output row r,
   * and y and part hold M / 2 rows                                        */
  int32_t pairs;
  int32_t tiles_m, tiles_n;   /* output tile grid (256 x 256 kernels)     */
  /* split-K (256 x 256 kernels): workgroup = (K slice, tile); slice sp
   * covers K [sp * kslice, (sp + 1) * kslice) and, when splits > 1, writes
   * f32 partial sums to part [splits, M, N] instead of y                  */
  float* part;
  int32_t kslice, splits;
} rlxq_gemm_args;


#endif
