/*
 * rlxq_oracle.h -- CPU restatement of rlx-models' quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing on the product path may link, load or
 * call this code: it is the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP library against.
 *
 * The reference's own arithmetic lives in external Rust crates (rlx-cpu,
 * rlx-gguf, rlx-mlx-io 0.2.19) that are not part of /root/reference and cannot
 * be built here.  Every function below restates an algorithm that the
 * reference states in-repo, cited at file:line, or the public GGML block
 * format the reference's loaders hand to those crates.  How each function is
 * pinned (known-answer vectors from the reference's tests, closed forms,
 * brute force) is recorded beside its test in tests/test_oracle.py.
 *
 * Pinning status per function:
 *   f16/bf16 conversions ........ pinned (exhaustive cross-check vs numpy)
 *   quantize/dequantize Q8_0 .... pinned (flint quant.rs round trips, KATs)
 *   quantize/dequantize Q4_0 .... pinned (gguf_legacy_quant_matmul.rs KAT,
 *                                  flint representable-block round trip)
 *   quantize/dequantize Q4_1 .... closed form pinned; the byte order of the
 *                                  nibbles follows the public GGML block_q4_1
 *                                  layout (no reference code in the tree fixes
 *                                  it): "parity unpinned" at the byte level.
 *   dequantize Q4_K ............. the public GGML block_q4_K layout (256-weight
 *                                  super-blocks, 6-bit scales and mins); the
 *                                  reference calls rlx_gguf::dequant_q4_k, which
 *                                  is absent: pinned by closed forms and bit-level
 *                                  probes of the scale packing, "parity unpinned"
 *                                  against reference code.
 *   dequantize Q6_K ............. the public GGML block_q6_K layout (ql / qh /
 *                                  int8 scales per 16 weights / f16 d); absent
 *                                  rlx_gguf::dequant_q6_k: pinned by bit probes
 *                                  of the code layout and closed forms, "parity
 *                                  unpinned" against reference code.
 *   MLX affine dequant .......... pinned (mlx_dequant.rs:100-110 KAT,
 *                                  mlx_affine.rs:290-330 matmul test)
 *   matmul / grouped / MoE ...... pinned (closed forms, f64 brute force,
 *                                  quant_parity_backends.rs structure)
 *   int8 activation / weight quant pinned (bitnet.rs:76-93 and
 *                                  common.rs:466-482 closed forms)
 */
#ifndef RLXQ_ORACLE_H
#define RLXQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scheme ids: the same numbering as include/rlxq.h. */
enum {
    ORC_GGUF_Q8_0 = 1,
    ORC_GGUF_Q4_0 = 2,
    ORC_GGUF_Q4_1 = 3,
    ORC_MLX_AFFINE4 = 4,
    ORC_MLX_AFFINE8 = 5,
    ORC_INT8_BLOCK = 6,
    ORC_GGUF_Q4_K = 7,
    ORC_GGUF_Q6_K = 8,
    ORC_GGUF_Q5_K = 10,
    ORC_GGUF_Q3_K = 11,
    ORC_GGUF_Q2_K = 12,
    ORC_GGUF_Q8_K = 13,
};

/* ---- scalar conversions (IEEE binary16 / bfloat16, round to nearest even) */
uint16_t orc_f32_to_f16(float v);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float v);
float orc_bf16_to_f32(uint16_t b);
void orc_f32_to_f16_n(const float* src, int64_t n, uint16_t* dst);
void orc_f16_to_f32_n(const uint16_t* src, int64_t n, float* dst);
void orc_f32_to_bf16_n(const float* src, int64_t n, uint16_t* dst);
void orc_bf16_to_f32_n(const uint16_t* src, int64_t n, float* dst);

/* ---- GGUF legacy block codecs (32 weights per block) -------------------- */
int64_t orc_block_bytes(int scheme);           /* 34 / 18 / 20; K-quants 144 (Q4_K) / 210 (Q6_K) /
                                                  176 (Q5_K) / 110 (Q3_K) / 84 (Q2_K) / 292 (Q8_K); else -1 */
int64_t orc_block_len(int scheme);             /* weights per block: 32, or 256 (the K-quants) */
int64_t orc_row_bytes(int scheme, int64_t k);  /* k/len * block bytes, else -1 */
/* Quantize n (multiple of 32) floats into packed blocks. 0 on success. */
int orc_quantize(int scheme, const float* src, int64_t n, uint8_t* dst);
/* Dequantize n (multiple of 32) weights. 0 on success. */
int orc_dequantize(int scheme, const uint8_t* src, int64_t n, float* dst);
/* Q4_K / Q5_K: the 6-bit (scale, min) of sub-block s (0..7) from the 12 packed bytes. */
void orc_q4k_scale_min(const uint8_t* q, int s, int* sc, int* mn);
/* Q3_K: the 6-bit scale of 16-weight group s (0..15) from the 12 packed bytes
 * (unsigned, 0..63; the weight uses scale - 32). */
int orc_q3k_scale(const uint8_t* q, int s);

/* ---- MLX affine (LSB-first u32 packing, w = scale*code + bias) ---------- */
/* Pack row-major codes [rows, cols] into u32 words, LSB-first. */
int orc_mlx_pack(const uint32_t* codes, int64_t rows, int64_t cols, int bits,
                 uint32_t* dst);
/* Dequantize with f32 scales/biases [rows, cols/group]. */
int orc_mlx_dequantize(const uint32_t* wq, const float* scales,
                       const float* biases, int64_t rows, int64_t cols,
                       int bits, int group, float* dst);

/* ---- dense DequantMatMul: y[m,n] = sum_k x[m,k] * W[n,k] ---------------- */
/* Truth: dequantize, then accumulate in double. y is written as double. */
int orc_matmul_f64(int scheme, const float* x, const uint8_t* w, int64_t m,
                   int64_t k, int64_t n, double* y);
/* Reference-order f32 (flint quant.rs:250-292 block dot: 8 lanes of mul_add,
 * then sum = d.mul_add(lane sum, sum)); Q4_1 adds m * (block sum of x). */
int orc_matmul_refl(int scheme, const float* x, const uint8_t* w, int64_t m,
                    int64_t k, int64_t n, float* y);
/* Same, rows partitioned over nthreads OpenMP threads (0 = all). */
int orc_matmul_refl_par(int scheme, const float* x, const uint8_t* w,
                        int64_t m, int64_t k, int64_t n, float* y,
                        int nthreads);
/* MLX affine, f64 accumulate over dequantized weights. */
int orc_mlx_matmul_f64(const float* x, const uint32_t* wq, const float* scales,
                       const float* biases, int64_t m, int64_t k, int64_t n,
                       int bits, int group, double* y);

/* ---- grouped expert matmul (Op::DequantGroupedMatMul) -------------------- */
/* out[r,:] = x[r,:] . dequant(bank[e[r]])^T, bank = E contiguous [N,K] slabs,
 * expert_idx carried as F32 like the IR.  f64 accumulate. */
int orc_grouped_matmul_f64(int scheme, const float* x, const uint8_t* bank,
                           const float* expert_idx, int64_t rows, int64_t k,
                           int64_t n, int64_t num_experts, double* y);

/* ---- MoE routing ------------------------------------------------------- */
/* Row softmax then top-k (descending probability, ties to lower index).
 * ids/probs are [rows, k]; renorm != 0 divides by the kept mass. */
int orc_topk_softmax(const float* logits, int64_t rows, int64_t e, int64_t k,
                     int renorm, int32_t* ids, float* probs);
/* y[r,:] = sum_j probs[r,j] * (x[r,:] . W[ids[r,j]]^T), f64 accumulate. */
int orc_moe_f64(int scheme, const float* x, const uint8_t* bank,
                const int32_t* ids, const float* probs, int64_t rows,
                int64_t topk, int64_t k, int64_t n, int64_t num_experts,
                double* y);

/* ---- int8 paths --------------------------------------------------------- */
/* bitnet.rs:76-93: per row s = amax/127 (1 if 0), q = round(x/s) clamp 127.
 * (round half away from zero, like f32::round.) */
int orc_quantize_act_int8(const float* x, int64_t rows, int64_t cols,
                          int8_t* q, float* scales);
/* common.rs:466-482: per output channel of a [k,n] row-major weight. */
int orc_quantize_int8_col(const float* w, int64_t k, int64_t n, int8_t* q,
                          float* scales);
/* W8A8: y[m,n] = (sum_k qx[m,k]*qw[k,n]) * sx[m] * sw[n]; int32 exact sum. */
int orc_w8a8_matmul(const int8_t* qx, const float* sx, const int8_t* qw,
                    const float* sw, int64_t m, int64_t k, int64_t n,
                    float* y);
/* Int8Block weight-only (int8_kernel.rs:59-89): y = x . ((Wq - zp) * s),
 * Wq [k,n] row-major, f64 accumulate. */
int orc_int8_block_matmul_f64(const float* x, const int8_t* wq,
                              const float* scale, const float* zp, int64_t m,
                              int64_t k, int64_t n, double* y);

#ifdef __cplusplus
}
#endif
#endif
