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
  /* exact kernels with f32 activations: M counts x16 rows prepared in
   * blocks of 64, rows 64b .. 64b + 31 the f16 rounding of rows 32b .. 32b
   * + 31 (hi) and rows 64b + 32 .. the remainders (lo); y and part hold
   * m_out rows                                                            */
  int32_t pairs;
  int64_t m_out;
  int32_t tiles_m, tiles_n;   /* output tile grid (256 x 256 kernels)     */
  /* split-K (256 x 256 kernels): workgroup = (K slice, tile); slice sp
   * covers K [sp * kslice, (sp + 1) * kslice) and, when splits > 1, writes
   * f32 partial sums to part [splits, M, N] instead of y                  */
  float* part;
  int32_t kslice, splits;
} rlxq_gemm_args;


#endif
