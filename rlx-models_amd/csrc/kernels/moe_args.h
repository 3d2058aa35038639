/* Argument blocks of the grouped-expert kernels, shared by the host (g++)
 * and device (hipcc) compilers: plain C types only. */
#ifndef RLXQ_MOE_ARGS_H
#define RLXQ_MOE_ARGS_H
#include <stdint.h>

/* Routing table in scratch memory (int32):
 *   [0]                      number of fired experts F
 *   [1, 1 + E)               fired expert ids, slots 0..F-1
 *   [1 + E, 2 + 2E)          entry offsets per slot, F + 1 valid
 *   [2 + 2E, 2 + 2E + n)     entry ids grouped by slot
 * An entry is one (token row, top-k slot) pair: entry = row * top_k + slot. */
typedef struct rlxq_moe_table_args {
  const int32_t* ids;     /* [n] int32 expert ids, or NULL               */
  const float* idx_f32;   /* [n] f32 expert ids (IR form), or NULL       */
  int32_t* table;         /* routing table, 2 + 2E + n int32             */
  void* zero_rows;        /* rows of invalid entries are zeroed here     */
  int64_t n, N, zero_ld;  /* entries, row length, row stride of zero_rows */
  int32_t E, zero_bf16;
} rlxq_moe_table_args;

typedef struct rlxq_moe_gemv_args {
  const void* x;          /* activations                                  */
  const uint8_t* bank;    /* E contiguous [N, K] packed slabs             */
  const void* scales;     /* MLX: [E, N, K/group], else NULL              */
  const void* biases;
  const int32_t* table;   /* routing table (see above)                   */
  void* y;                /* output rows, leading dimension y_ld          */
  int64_t N, rb, y_ld, x_ld;
  int32_t K, E, group, sb_bf16, y_bf16;
  int32_t x_div;          /* activation row of entry = entry / x_div      */
  int32_t tiles_n;        /* row tiles per expert                         */
  int32_t tile_rows;      /* weight rows per tile: 64, 128, 192 or 256    */
  int32_t swiglu;         /* 1: rows [0, N/2) gate, [N/2, N) up; y [entries, N/2]
                             = silu(x.Wg^T) * (x.Wu^T)                     */
  /* routing built in each workgroup (small entry counts): expert of each of
   * the n_entries entries as int32 ids or f32 indices (one of them); the
   * table above is then unused                                             */
  const int32_t* ids;
  const float* idx_f32;
  int32_t n_entries;
  /* COMBINE in the same launch (register kernels, routing in the
   * workgroups): y above holds the per-entry rows; the workgroup that
   * completes a (token row, tile) sums that row's top_k entry rows in slot
   * order, weighted by probs [rows, top_k], into out [rows, N] (entries with
   * an invalid expert id contribute nothing).  counters [rows, tiles_n] are
   * zero on entry and left at zero.  counters == NULL: no combine here.   */
  const float* probs;
  void* out;
  int32_t* counters;
  int32_t top_k, out_bf16;
} rlxq_moe_gemv_args;

/* Grouped batched-decode MFMA path (prefill-sized MoE calls): the entries of
 * each fired expert (table order) are laid out in gathered activation rows,
 * each expert's run padded to whole chunks of rows_per_chunk rows.
 * rlxq_moe_pad_k writes cmap ([0]: chunks, [1 + c]: expert of chunk c) and
 * emap ([Mp]: entry of gathered row, -1 for padding).                     */
typedef struct rlxq_moe_pad_args {
  const int32_t* table;
  int32_t* cmap;
  int32_t* emap;
  int64_t Mp;
  int32_t E, rows_per_chunk;
} rlxq_moe_pad_args;

typedef struct rlxq_moe_sk_args {
  const uint16_t* x16;    /* gathered f16 rows, fragment-major over Mp    */
  const float* inv_s;     /* [Mp] factors undoing the row scaling         */
  const int32_t* cmap;
  const int32_t* emap;
  const uint8_t* bank;    /* E contiguous [N, K] packed slabs             */
  void* y;                /* entry rows, leading dimension y_ld           */
  int64_t N, K, rb, y_ld, Mp;
  int32_t tiles_n, y_bf16;
  int32_t swiglu;         /* 1: rows [0, N/2) gate, [N/2, N) up; y [entries, N/2]
                             = silu(x.Wg^T) * (x.Wu^T)                     */
  /* pairs: the x16 rows are hi/lo pairs (row 2r + 1 the remainder of row
   * 2r, both of gathered row r, whose entry is emap[r]); the epilogue adds
   * each pair                                                             */
  int32_t pairs;
  /* MLX affine: per-group scales and biases [E, N, K / group] (f32, or bf16
   * where sb_bf16 == 1); MXFP4: E8M0 bytes [E, N, K / 32] (sb_bf16 == 2);
   * unused by the GGUF formats (group 32)                                 */
  const void* scales;
  const void* biases;
  int64_t group;
  int32_t sb_bf16, pad2;
  const float* ssum;      /* block sums of x16 (min / bias formats)       */
} rlxq_moe_sk_args;

#endif
