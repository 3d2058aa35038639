/* Argument blocks of the batched-decode ("skinny", small M) kernels, shared
 * by the host (g++) and device (hipcc) compilers: plain C types only. */
#ifndef RLXQ_SKINNY_ARGS_H
#define RLXQ_SKINNY_ARGS_H
#include <stdint.h>

/* Activation preparation: x [M, K] (f32 or bf16) -> x16 f16 (or bf16) scaled by a
 * power of two per row (inv_s[m] = 1 / scale) and permuted within each
 * 32-element block to the order the packed codes unpack to.  Row-major
 * [M, K], or (frag_major) fragment-major over Mp >= M rows (rows M .. Mp - 1
 * zero): the 16-byte piece i (positions 8i .. 8i + 7) of block 4c + g of row
 * m at piece ((4c + i) * Mp + m) * 4 + g, so the MFMA A fragments of 16 rows
 * are 1 KB of contiguous memory. */
typedef struct rlxq_x16_args {
  const void* x;
  uint16_t* x16;
  float* inv_s;
  int64_t M, K, Mp;
  int32_t x_bf16;
  int32_t nibble_order;   /* 0 natural, 1 GGUF nibbles, 2 MLX nibbles    */
  int32_t frag_major, rdiv;
  /* gathered rows (fragment-major only): x16 row r is x row rmap[r] / rdiv,
   * a zero row where rmap[r] < 0; NULL: x16 row r is x row r             */
  const int32_t* rmap;
  int32_t out_bf16;       /* x16 holds bf16 (MXFP4's bf16 MFMA), not f16  */
  /* split: f32 rows in two parts, the rounded row (hi) and what that
   * rounding left over (lo, on the same scale), so that hi + lo carries ~22
   * (f16) or ~16 (bf16) significant bits of each f32 element; M counts the
   * rows of x (and rmap its entries), Mp the x16 rows.  split 1: x16 rows
   * 2r (hi) and 2r + 1 (lo) for row r; split 2 (row-major only): blocks of
   * 64 x16 rows, 64b + i the hi and 64b + 32 + i the lo part of row 32b + i
   * (rows past M zero)                                                      */
  int32_t split;
  /* inv_s[r] carries an extra factor 2^post_exp: the MLX affine kernels'
   * f16 weights are 2^8 times the true ones (post_exp = -8), so that group
   * scales down to ~2^-22 stay normal in f16                               */
  int32_t post_exp;
  /* fragment-major only, NULL for none: the sum of each prepared 32-element
   * block (f32, in the order the prepared values sum) at
   * ((b / 4) Mp + r) 4 + b % 4 for block b of x16 row r (0 for padding rows) */
  float* ssum;
} rlxq_x16_args;

typedef struct rlxq_skinny_args {
  const uint16_t* x16;    /* prepared activations [M, K] f16              */
  const float* inv_s;     /* [M]                                          */
  const uint8_t* w;       /* packed rows, row stride rb bytes             */
  float* part;            /* [splits, M, N] partial sums (splits > 1)     */
  void* y;                /* [M, N] output (splits == 1)                  */
  int64_t M, N, K, rb, y_ld;
  int64_t Mp;             /* rows of the fragment-major x16 (>= M)        */
  int32_t kslice;         /* K per split, a multiple of 128               */
  int32_t splits, tiles_n, y_bf16;
  /* MLX affine 4-bit: per-group scales and biases [N, K / group] (f32, or
   * bf16 where sb_bf16 == 1); MXFP4: E8M0 scale bytes [N, K / 32]
   * (sb_bf16 == 2); unused by the GGUF formats                           */
  const void* scales;
  const void* biases;
  int64_t group;
  int32_t sb_bf16;
  /* pairs: M counts x16 rows prepared with split (row 2r hi, 2r + 1 lo of
   * output row r); the epilogue adds each pair, and y and part hold M / 2
   * rows                                                                  */
  int32_t pairs;
  /* block sums of x16 (rlxq_x16_args.ssum): the formats with a min / bias  */
  const float* ssum;
} rlxq_skinny_args;

#endif
