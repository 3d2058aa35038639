/*
 * rlxq.h -- C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * One shared library (librlxq.so) with its gfx950 code object built in.  It
 * replaces the backend kernel behind rlx-models' group-wise packed-weight
 * linear op and its grouped-expert siblings.  Every entry point is plain C:
 * pointers, sizes and an opaque stream, no C++ or torch types.
 *
 * Conventions shared by every entry point
 *   - Device pointers (x, w, scales, biases, y, expert_idx, ids, probs) are
 *     owned by the caller and must stay valid until the stream has run the
 *     call.  `stream` is a hipStream_t passed as void* (NULL = null stream).
 *   - W is logically [N, K] row-major, K contiguous, and y = x . W^T, as in
 *     `Op::DequantMatMul` (crates/rlx-models-core/src/standard_decoder.rs:727-738,
 *     crates/rlx-qwen3/src/precision.rs:98-112).  Int8Block weights are
 *     [K, N] like the reference's (crates/rlx-kimi-k3/examples/int8_kernel.rs:59-89).
 *   - Results are written with fp32 accumulation.  The reference's output is
 *     always F32; RLXQ_BF16 output (round to nearest even) is offered for
 *     prefill callers.
 *   - Return value: RLXQ_OK (0) or a negative rlxq_status.  Shape, scheme,
 *     dtype, alignment and null-pointer problems are rejected on the host
 *     before any kernel is launched; rlxq_last_error() names the argument.
 *   - A context is used by one host thread at a time (the reference's
 *     CompiledGraph is &mut self); calls on different streams may overlap
 *     (the library's scratch is kept per stream).
 *   - Scratch: some paths (batched decode, split-K, MoE routing, W8A8) use
 *     device scratch that the context allocates per stream and grows on
 *     demand, by at least half its size each time (so the buffers growth
 *     replaces total less than twice the live one).  A replaced buffer that
 *     was never used under stream capture is freed by a later call on the
 *     stream once the work queued before its replacement has finished; one
 *     that was used under capture is kept until rlxq_release_stream or
 *     rlxq_destroy, so a HIP graph captured earlier stays valid.  A call
 *     under stream capture must not need growth (the
 *     allocation fails under global capture): size the stream's scratch
 *     first with rlxq_reserve_workspace, or run the call once uncaptured.
 *     The MoE combine fused into the down launch (when selected) also
 *     takes 64 KB of per-stream counters, zeroed once when first used (or
 *     by rlxq_reserve_workspace) and left at zero by every call.
 */
#ifndef RLXQ_H
#define RLXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight schemes.  Names mirror rlx_ir::quant::QuantScheme variants. */
typedef enum rlxq_scheme {
    RLXQ_GGUF_Q8_0 = 1,   /* GgufQ8_0: 34 B / 32 w: f16 d, 32 x i8; w = d*q      */
    RLXQ_GGUF_Q4_0 = 2,   /* GgufQ4_0: 18 B / 32 w: f16 d, 16 B nibbles; d*(q-8) */
    RLXQ_GGUF_Q4_1 = 3,   /* GgufQ4_1: 20 B / 32 w: f16 d, f16 m, nibbles; d*q+m */
    RLXQ_MLX_AFFINE4 = 4, /* MlxAffine{bits:4, group_size}: u32 LSB-first codes,
                             scale*code + bias, scales/biases [N, K/group]       */
    RLXQ_MLX_AFFINE8 = 5, /* MlxAffine{bits:8, group_size}                       */
    RLXQ_INT8_BLOCK = 6,  /* Int8Block{block_size: K}: i8 [K, N], scale [N],
                             zp [N] (NULL = 0); y = x . ((Wq - zp) * scale)      */
    RLXQ_GGUF_Q4_K = 7,   /* GgufQ4K (weight_loader.rs:502; host twin
                             rlx_gguf::dequant_q4_k, crates/rlx-sam3/src/
                             packed_gguf.rs:50): 144 B / 256 w: f16 d, f16 dmin, 12 B of
                             6-bit scales/mins, 128 nibble bytes;
                             w = (d*sc)*q - dmin*mn.  Dense and grouped ops,
                             dequantize; K % 256 == 0, w 16-byte aligned       */
    RLXQ_GGUF_Q6_K = 8,   /* GgufQ6K (weight_loader.rs maps GgmlType::Q6K;
                             host twin rlx_gguf::dequant_q6_k, crates/rlx-sam3/
                             src/packed_gguf.rs): 210 B / 256 w: ql[128],
                             qh[64], int8 scales[16], f16 d;
                             w = (d*scale)*(code - 32).  Dense (GEMV family)
                             and grouped ops, dequantize; K % 256 == 0        */
    RLXQ_MLX_MXFP4 = 9,   /* MlxMxfp4{group_size: 32} (crates/rlx-models-core/
                             src/mxfp4_pack.rs:16-50): codes [N, K/2], two E2M1
                             codes per byte, low nibble = even element; one
                             scale per 32: E8M0 bytes [N, K/32] (RLXQ_U8, the
                             dense op's operand; 2^(b-127), b = 0 -> 0) or the
                             decoded value as BF16 (the grouped op's [E, N, G]
                             operand).  No bias (biases are not read).
                             w = E2M1(code) * scale.  GEMV family, grouped ops
                             and dequantize                                    */
    /* The other K-quants of the reference's DeviceMatmul table
     * (crates/rlx-laguna/src/device_matmul.rs:64-76) and of its GGUF scheme
     * map (crates/rlx-models-core/src/weight_loader.rs:497-505; host twins
     * rlx_gguf::dequant_q5_k / q3_k / q2_k / q8_k, crates/rlx-sam3/src/
     * packed_gguf.rs:46-56).  256 weights per super-block, K % 256 == 0; the
     * GEMV family (every M), grouped ops and dequantize.                     */
    RLXQ_GGUF_Q5_K = 10,  /* 176 B: f16 d, f16 dmin, the 12 Q4_K scale bytes,
                             qh[32], qs[128]; code = nibble | qh bit << 4;
                             w = (d*sc)*code - dmin*mn; w 16-byte aligned      */
    RLXQ_GGUF_Q3_K = 11,  /* 110 B: hmask[32], qs[64], 12 B of sixteen 6-bit
                             scales, f16 d; code = 2 bits - (hmask bit ? 0 : 4);
                             w = (d*(scale-32))*code; w 4-byte aligned (its
                             110-byte rows are 2-byte aligned)                */
    RLXQ_GGUF_Q2_K = 12,  /* 84 B: scales[16] (scale | min << 4), qs[64], f16
                             d, f16 dmin; w = (d*sc)*code - dmin*mn;
                             w 4-byte aligned                                  */
    RLXQ_GGUF_Q8_K = 13   /* 292 B: f32 d, int8 qs[256], int16 bsums[16];
                             w = d*q; w 4-byte aligned                         */
} rlxq_scheme;

/* Element types of activations, outputs and MLX scale/bias slabs. */
typedef enum rlxq_dtype {
    RLXQ_F32 = 0,
    RLXQ_BF16 = 1,
    RLXQ_U8 = 2           /* raw bytes: MXFP4's E8M0 scale slab              */
} rlxq_dtype;

typedef enum rlxq_status {
    RLXQ_OK = 0,
    RLXQ_E_NULL = -1,     /* a required pointer is NULL                      */
    RLXQ_E_SHAPE = -2,    /* m/k/n/rows/experts out of range or inconsistent */
    RLXQ_E_SCHEME = -3,   /* unknown scheme, or not valid for this call     */
    RLXQ_E_ALIGN = -4,    /* pointer or K not aligned as the scheme needs   */
    RLXQ_E_DTYPE = -5,    /* unsupported activation / output dtype          */
    RLXQ_E_HIP = -6,      /* a HIP runtime call failed                      */
    RLXQ_E_NOMEM = -7,    /* device or host allocation failed               */
    RLXQ_E_INDEX = -8,    /* expert index outside [0, num_experts)          */
    RLXQ_E_NOKERNEL = -9, /* code object lacks the kernel for this variant  */
    RLXQ_E_DEVICE = -10,  /* device is not gfx950 or does not exist         */
    RLXQ_E_IO = -11,      /* a checkpoint file cannot be opened or read     */
    RLXQ_E_FORMAT = -12,  /* a checkpoint file is not valid GGUF            */
    RLXQ_E_NOTFOUND = -13,/* no tensor or metadata key of that name         */
    RLXQ_E_TAKEN = -14,   /* the weight was already taken                   */
    RLXQ_E_SCRATCH = -15  /* call needs more scratch than the no-allocation
                             entry point holds (RLXQ_NOALLOC_SCRATCH_BYTES)  */
} rlxq_status;

typedef struct rlxq_ctx rlxq_ctx;

/* Context: loads the embedded gfx950 code object on `device` with
 * hipModuleLoadData and resolves every kernel.  Replaces the per-backend
 * setup behind Session::new(Device::Rocm) (external rlx-runtime; caller
 * crates/rlx-laguna/src/device_matmul.rs:94-111 `DeviceMatmul::try_new`). */
int rlxq_init(int device, rlxq_ctx** out);
int rlxq_destroy(rlxq_ctx* ctx);
const char* rlxq_strerror(int status);
/* Detail of the last failure on this context (empty if none). */
const char* rlxq_last_error(const rlxq_ctx* ctx);
/* Name of the last kernel this context launched (diagnostics and profiling;
 * no counterpart in the reference). */
const char* rlxq_last_kernel(const rlxq_ctx* ctx);
/* Library version string, e.g. "rlxq 0.1.0 gfx950". */
const char* rlxq_version(void);
/* Scratch management (no counterpart in the reference, whose runtime owns
 * its arena): make the scratch of `stream` at least `bytes` (and create
 * its zeroed counters); report its
 * size (0 if the stream has none); and free every scratch buffer the stream
 * holds after waiting for the stream (graphs that captured calls on it must
 * not be replayed afterwards).  For callers that capture graphs or use many
 * streams (per-request streams, torch's stream pool). */
int rlxq_reserve_workspace(rlxq_ctx* ctx, void* stream, size_t bytes);
int64_t rlxq_workspace_bytes(const rlxq_ctx* ctx, void* stream);
/* Bytes of replaced scratch buffers the stream still holds (not yet freed). */
int64_t rlxq_workspace_retired_bytes(const rlxq_ctx* ctx, void* stream);
int rlxq_release_stream(rlxq_ctx* ctx, void* stream);

/* Dense DequantMatMul: y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
 * Replaces the backend kernel of Op::DequantMatMul{scheme} (the IR op is
 * emitted at crates/rlx-models-core/src/standard_decoder.rs:727-738 and
 * crates/rlx-qwen3/src/precision.rs:98-112; host twin
 * rlx_cpu::gguf_matmul::gguf_matmul_bt, call sites
 * crates/rlx-laguna/src/packed_forward.rs:30,233-241).
 *   GGUF schemes ("Packed2"): w = packed blocks, N rows of K/32 blocks;
 *     scales = biases = NULL, group_size ignored.  K % 64 == 0 for Q8_0 and
 *     Q4_0 (block pairs are read dword aligned), K % 32 == 0 for Q4_1.
 *   MLX affine ("Affine4"): w = u32 codes [N, K*bits/32]; scales/biases
 *     [N, K/group_size] of `sb_dtype`; group_size in {32, 64, 128}.
 *   Int8Block: w = i8 [K, N]; scales = f32 [N]; biases = zp f32 [N] or NULL.
 * x: [M, K] of x_dtype; y: [M, N] of y_dtype. */
int rlxq_dequant_matmul(rlxq_ctx* ctx, int scheme, int group_size,
                        const void* x, int x_dtype, const void* w,
                        const void* scales, const void* biases, int sb_dtype,
                        int64_t m, int64_t k, int64_t n, void* y, int y_dtype,
                        void* stream);

/* The dense op for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments, kernels and results as
 * rlxq_dequant_matmul, but it calls no hipMalloc / hipFree: the scratch that
 * batched decode and split-K need is a static device array of
 * RLXQ_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  A call
 * that would need more returns RLXQ_E_SCRATCH before any launch.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, contexts or threads) race and must be serialised by the caller. */
#define RLXQ_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int rlxq_dequant_matmul_noalloc(rlxq_ctx* ctx, int scheme, int group_size,
                                const void* x, int x_dtype, const void* w,
                                const void* scales, const void* biases,
                                int sb_dtype, int64_t m, int64_t k, int64_t n,
                                void* y, int y_dtype, void* stream);

/* Grouped expert DequantMatMul: out[r, :] = x[r, :] . dequant(bank[e[r]])^T.
 * Replaces Op::DequantGroupedMatMul{scheme} (crates/rlx-qwen35/src/builder.rs:2955-2973;
 * host twin rlx_cpu::gguf_matmul::gguf_grouped_matmul_bt_fused, call site
 * crates/rlx-laguna/src/packed_forward.rs:583-623) and, for MLX schemes,
 * Op::DequantGroupedMatMulMlx (standard_decoder.rs:12731-12760, bf16 scale
 * slabs [E, N, K/group]).  bank = E contiguous [N, K] slabs; expert_idx is
 * F32 [rows] like the IR's TopK output.  The rows are routed on the device:
 * each fired expert's weights are streamed once for all of its rows.  The
 * indices live on the device, so they are not read back: a row whose index
 * is not an integer in [0, num_experts) gets a zero output row (the host
 * session API below validates host indices and returns RLXQ_E_INDEX). */
int rlxq_dequant_grouped_matmul(rlxq_ctx* ctx, int scheme, int group_size,
                                const void* x, int x_dtype, const void* bank,
                                const void* scales, const void* biases,
                                int sb_dtype, const float* expert_idx,
                                int64_t rows, int64_t k, int64_t n,
                                int64_t num_experts, void* y, int y_dtype,
                                void* stream);

/* MoE routed-expert grouped GEMV, routed on the device from ids [rows, top_k]
 * (int32).  Modes, which together make one expert FFN
 * (crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:338-373 and
 * standard_decoder.rs:12612-12760):
 *   RLXQ_MOE_EXPAND : x [rows, K] -> y [rows*top_k, N],
 *                     y[r*top_k + j] = x[r] . W[ids[r, j]]^T   (probs unused)
 *   RLXQ_MOE_COMBINE: x [rows*top_k, K] -> y [rows, N],
 *                     y[r] = sum_j probs[r, j] * (x[r*top_k + j] . W[ids[r, j]]^T)
 *   RLXQ_MOE_EXPAND_SWIGLU: the fused gate|up projection with its SwiGLU
 *                     (the GroupedSwiglu graph, crates/rlx-laguna/src/device_matmul.rs:383-426):
 *                     expert slabs hold gate rows [0, N/2) then up rows
 *                     [N/2, N); y [rows*top_k, N/2] = silu(g) * u with
 *                     g, u = x[r] . W^T rows, silu(g) = g / (1 + exp(-g))
 * GGUF schemes only, K-quants included (scales/biases NULL).  An id outside [0, num_experts)
 * gives a zero output row (EXPAND) or a zero contribution (COMBINE). */
typedef enum rlxq_moe_mode {
    RLXQ_MOE_EXPAND = 0,
    RLXQ_MOE_COMBINE = 1,
    RLXQ_MOE_EXPAND_SWIGLU = 2
} rlxq_moe_mode;
int rlxq_moe_grouped(rlxq_ctx* ctx, int scheme, int mode, const void* x,
                     int x_dtype, const void* bank, const int32_t* ids,
                     const float* probs, int64_t rows, int64_t top_k,
                     int64_t k, int64_t n, int64_t num_experts, void* y,
                     int y_dtype, void* stream);

/* Peak probes for the measurement (no counterpart in the reference: they
 * give the bench its measured denominators besides the data-sheet peaks).
 *   kind RLXQ_PROBE_MFMA (0): `work` rounds of four independent
 *     v_mfma_f32_32x32x16_bf16 per wave on register operands, 8 workgroups
 *     of 4 waves per CU; *count = the flops issued.
 *   kind RLXQ_PROBE_READ (1): every byte of `buf` [work bytes, 16-byte
 *     aligned, a multiple of 4096] read once with 16-byte loads, a
 *     grid-stride loop over 8 workgroups per CU; *count = work.
 *   kind RLXQ_PROBE_READ4 (2): the same bytes with the grid sized to them,
 *     four independent 16-byte loads per thread (work <= 1 GiB): the
 *     load-only floor of a small weight stream.
 *   kind RLXQ_PROBE_TILE20 (3): `buf` [work bytes, a multiple of 81920,
 *     at most 65536 x 81920]
 *     as rows of 2560 bytes (4096 Q4_1 codes) read with the register-
 *     streamed batched-decode kernel's lane pattern and no arithmetic: per
 *     wave instruction 16 rows x 80 bytes, one 20-byte block per lane;
 *     *count = work.
 * sink: device memory of at least max(8 x CUs, 65536) x 4 bytes, written only
 * to keep the work live.  Time the call with events on `stream`. */
#define RLXQ_PROBE_MFMA 0
#define RLXQ_PROBE_READ 1
#define RLXQ_PROBE_READ4 2
#define RLXQ_PROBE_TILE20 3
int rlxq_peak_probe(rlxq_ctx* ctx, int kind, const void* buf, int64_t work, void* sink, int64_t* count,
                    void* stream);

/* Router: row softmax of logits [rows, E] (f32), top-k by probability
 * (ties to the lower expert id), optional renormalisation of the kept
 * probabilities (norm_topk_prob, standard_decoder.rs:12634-12661).
 * E <= 1024, top_k <= 64.
 * Writes ids [rows, top_k] int32 and probs [rows, top_k] f32. */
int rlxq_moe_route(rlxq_ctx* ctx, const float* logits, int64_t rows,
                   int64_t num_experts, int64_t top_k, int renorm,
                   int32_t* ids, float* probs, void* stream);

/* SwiGLU between the fused gate|up projection and down: for each row,
 * out[i] = silu(gu[i]) * gu[inter + i], gu [rows, 2*inter] -> out [rows, inter]
 * (crates/rlx-laguna/src/device_matmul.rs:383-426 GroupedSwiglu graph). */
int rlxq_swiglu(rlxq_ctx* ctx, const void* gu, int gu_dtype, int64_t rows,
                int64_t inter, void* out, int out_dtype, void* stream);

/* W8A8 GEMM: per-row int8 activation quantisation computed on the fly
 * (crates/rlx-quant-calib/src/bitnet.rs:76-93) times per-channel int8
 * weights (crates/rlx-kimi-k3/src/common.rs:466-482, wq [K, N], w_scale [N])
 * on int8 MFMA with int32 accumulation: y = (sum qx*qw) * sx[m] * sw[n].
 * The reference has no such kernel; it has the two quantisers. */
int rlxq_w8a8_gemm(rlxq_ctx* ctx, const void* x, int x_dtype,
                   const int8_t* wq, const float* w_scale, int64_t m,
                   int64_t k, int64_t n, void* y, int y_dtype, void* stream);

/* The activation quantiser used by rlxq_w8a8_gemm, exposed for checking:
 * q [m, k] int8 and scales [m] f32. */
int rlxq_quantize_act_int8(rlxq_ctx* ctx, const void* x, int x_dtype,
                           int64_t m, int64_t k, int8_t* q, float* scales,
                           void* stream);

/* Dequantize `rows` packed rows of K weights to f32 [rows, K] with the same
 * arithmetic the kernels use (bit-exact against the CPU codec).  GGUF and
 * MLX schemes; MLX takes scales/biases as in rlxq_dequant_matmul. */
int rlxq_dequantize(rlxq_ctx* ctx, int scheme, int group_size, const void* w,
                    const void* scales, const void* biases, int sb_dtype,
                    int64_t rows, int64_t k, float* out, void* stream);

/* Bytes of one packed row of K weights for a GGUF scheme (-1 if invalid). */
int64_t rlxq_row_bytes(int scheme, int64_t k);

/* ---- Host-side session API ----------------------------------------------
 * Mirrors rlx-laguna's DeviceMatmul (crates/rlx-laguna/src/device_matmul.rs:
 * 82-296): host slices in, host f32 out, weights uploaded once per distinct
 * host pointer and length and kept resident (`uploaded_ptr`, :41-62,301-352),
 * shape mismatch and unknown scheme rejected (:129-146, :64-76). */
typedef struct rlxq_device_matmul rlxq_device_matmul;
int rlxq_dm_try_new(int device, rlxq_device_matmul** out);
void rlxq_dm_free(rlxq_device_matmul* dm);
const char* rlxq_dm_last_error(const rlxq_device_matmul* dm);
/* y[m*n] = x[m*k] . W^T, W = packed GGUF bytes [n, k] (w_len bytes). */
int rlxq_dm_matmul(rlxq_device_matmul* dm, const float* x, size_t x_len,
                   const uint8_t* w_bytes, size_t w_len, size_t m, size_t k,
                   size_t n, int scheme, float* y);
/* out[i] = x[i] . expert[expert_idx[i]]^T over a resident expert stack. */
int rlxq_dm_grouped_matmul(rlxq_device_matmul* dm, const float* x,
                           size_t x_len, const uint8_t* w_bytes, size_t w_len,
                           const float* expert_idx, size_t idx_len, size_t m,
                           size_t k, size_t n, size_t num_experts, int scheme,
                           float* y);
/* down(silu(gate(x)) * up(x)) per row with expert expert_idx[row]
 * (DeviceMatmul::grouped_swiglu, crates/rlx-laguna/src/device_matmul.rs:221-296,
 * graph :383-426): x [m, h]; gate and up stacks [E, inter, h], down stack
 * [E, h, inter], each packed GGUF with its own scheme; y [m, h].  Gate and up
 * of one scheme are kept as one gate|up bank on the device (one upload) and
 * run as one launch with the SwiGLU fused. */
int rlxq_dm_grouped_swiglu(rlxq_device_matmul* dm, const float* x,
                           size_t x_len, const float* expert_idx,
                           size_t idx_len, const uint8_t* w_gate,
                           size_t gate_len, int gate_scheme,
                           const uint8_t* w_up, size_t up_len, int up_scheme,
                           const uint8_t* w_down, size_t down_len,
                           int down_scheme, size_t m, size_t h, size_t inter,
                           size_t num_experts, float* y);
/* Number of weight uploads performed so far (re-upload is skipped when the
 * same host pointers and lengths come back; a gate|up bank counts once). */
int64_t rlxq_dm_upload_count(const rlxq_device_matmul* dm);

/* ---- GGUF checkpoints: the on-disk step in front of the kernels ---------
 * Replaces the reference's GgufLoader packed path
 * (crates/rlx-models-core/src/weight_loader.rs:1360-1486, type map :497-565;
 * container parser: external crate rlx_gguf ^0.2.19) and its streamed upload
 * (crates/rlx-qwen3/src/high_level_runner.rs:474-499).  GGUF versions 2 and 3.
 * Host code only, except rlxq_gguf_upload. */
typedef struct rlxq_gguf rlxq_gguf;
typedef struct rlxq_gguf_tensor {
    const char* name;       /* valid until rlxq_gguf_close                    */
    int32_t ggml_type;      /* ggml type id as stored (F32 0, Q4_0 2, Q4_1 3,
                               Q8_0 8, Q4_K 12, Q6_K 14, BF16 30, ...)        */
    int32_t n_dims;         /* 1..4                                           */
    int64_t dims[4];        /* as stored: innermost first (unused dims = 1)   */
    uint64_t offset;        /* absolute file offset of the tensor's bytes     */
    int64_t nbytes;         /* -1 when the type has no fixed block layout here */
    int32_t scheme;         /* rlxq_scheme the kernels read it as, 0 = none   */
} rlxq_gguf_tensor;
/* Parse the header (the data is read on demand).  *out is set even when the
 * return is an error, so that rlxq_gguf_last_error can name the problem; the
 * handle is then only good for that and rlxq_gguf_close. */
int rlxq_gguf_open(const char* path, rlxq_gguf** out);
void rlxq_gguf_close(rlxq_gguf* g);
const char* rlxq_gguf_last_error(const rlxq_gguf* g);
int rlxq_gguf_version(const rlxq_gguf* g);
/* File offset of the aligned data section (general.alignment, default 32). */
int64_t rlxq_gguf_data_offset(const rlxq_gguf* g);
int64_t rlxq_gguf_tensor_count(const rlxq_gguf* g);
/* Index of the tensor, or RLXQ_E_NOTFOUND. */
int64_t rlxq_gguf_find_tensor(const rlxq_gguf* g, const char* name);
int rlxq_gguf_tensor_info(const rlxq_gguf* g, int64_t i, rlxq_gguf_tensor* info);
/* take_packed / take_packed_metadata (weight_loader.rs:1363-1486): the scheme
 * and the shape reversed to outermost first ([out, in] for a projection, as
 * the reference's `shape.reverse()`), and marks the weight taken; a second
 * take is RLXQ_E_TAKEN ("weight already taken").  A tensor stored in a form
 * the kernels do not read packed (F32, F16, BF16, other ggml types) gives
 * *scheme = 0 and RLXQ_OK and is not taken (the reference's Ok(None)).
 * Q4_1 always stays packed (the reference's RLX_GGUF_PACKED_Q4_1 opt-in
 * exists because its GPU backends cannot dequantise Q4_1). */
int rlxq_gguf_take_packed(rlxq_gguf* g, const char* name, int* scheme,
                          int64_t shape[4], int* n_dims, int64_t* nbytes);
/* The tensor's bytes as stored, into host memory of cap bytes (pread). */
int rlxq_gguf_read(rlxq_gguf* g, const char* name, void* dst, size_t cap);
/* The tensor's bytes as stored, into device memory of cap bytes: pread into
 * two 32 MiB pinned staging buffers, each copied on `stream` while the other
 * refills.  Returns when the last copy is queued; the bytes are on the device
 * once `stream` has run it.  The staging buffers live until rlxq_gguf_close. */
int rlxq_gguf_upload(rlxq_gguf* g, const char* name, void* dst, size_t cap,
                     void* stream);
/* Metadata: index of a key (or RLXQ_E_NOTFOUND), its name, its GGUF value
 * type (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
 * 9 array, 10 u64, 11 i64, 12 f64), element type and count (1 for a
 * scalar); element j as an integer, a float or a string (RLXQ_E_DTYPE when
 * the value is not of that kind). */
int64_t rlxq_gguf_meta_count(const rlxq_gguf* g);
int64_t rlxq_gguf_meta_find(const rlxq_gguf* g, const char* key);
const char* rlxq_gguf_meta_key(const rlxq_gguf* g, int64_t i);
int rlxq_gguf_meta_type(const rlxq_gguf* g, int64_t i, int* type,
                        int* elem_type, uint64_t* count);
int rlxq_gguf_meta_int(const rlxq_gguf* g, int64_t i, uint64_t j, int64_t* v);
int rlxq_gguf_meta_float(const rlxq_gguf* g, int64_t i, uint64_t j, double* v);
int rlxq_gguf_meta_str(const rlxq_gguf* g, int64_t i, uint64_t j,
                       const char** s, uint64_t* len);

/* ---- MLX checkpoints (mlx-community safetensors) --------------------------
 * Replaces the reference's MlxLoader and its take_packed_mlx
 * (crates/rlx-models-core/src/weight_loader.rs:906-1012, consumed by
 * load_proj, crates/rlx-models-core/src/standard_decoder.rs:590-645; reader
 * crate rlx-mlx-io, absent).  rlxq_mlx_open takes a checkpoint directory
 * (config.json with its "quantization" block, and model.safetensors.index.json
 * shards or every *.safetensors file) or one .safetensors file (config.json
 * from its directory when present).  Host code only, except rlxq_mlx_upload. */
typedef struct rlxq_mlx rlxq_mlx;
typedef enum rlxq_st_dtype {   /* safetensors element types */
    RLXQ_ST_BOOL = 1, RLXQ_ST_U8, RLXQ_ST_I8, RLXQ_ST_U16, RLXQ_ST_I16,
    RLXQ_ST_F16, RLXQ_ST_BF16, RLXQ_ST_U32, RLXQ_ST_I32, RLXQ_ST_F32,
    RLXQ_ST_U64, RLXQ_ST_I64, RLXQ_ST_F64, RLXQ_ST_F8_E4M3, RLXQ_ST_F8_E5M2
} rlxq_st_dtype;
typedef enum rlxq_mlx_mode {
    RLXQ_MLX_MODE_NONE = 0, RLXQ_MLX_MODE_AFFINE = 1, RLXQ_MLX_MODE_MXFP4 = 2
} rlxq_mlx_mode;
typedef struct rlxq_mlx_tensor {
    const char* name;       /* valid until rlxq_mlx_close                      */
    int32_t dtype;          /* rlxq_st_dtype                                   */
    int32_t n_dims;         /* 0..8                                            */
    int64_t shape[8];       /* outermost first (unused dims = 1)               */
    int64_t nbytes;
    const char* file;       /* the safetensors file holding it                 */
    uint64_t offset;        /* absolute file offset of its bytes               */
} rlxq_mlx_tensor;
/* A quantized Linear as the kernels read it (the reference's
 * MlxPackedLinear): codes [out, in * bits / 32] u32 LSB first, scales and
 * biases [out, in / group_size] of slab_dtype (BF16, F16 or F32; MXFP4: U8
 * E8M0 scales, no biases).  Tensor names point into the handle. */
typedef struct rlxq_mlx_packed {
    int32_t scheme;         /* RLXQ_MLX_AFFINE4 / 8, RLXQ_MLX_MXFP4; 0 = not packed */
    int32_t bits, group_size;
    int64_t out_features, in_features;
    const char* codes;
    const char* scales;
    const char* biases;     /* NULL for MXFP4                                  */
    int64_t codes_nbytes, scales_nbytes, biases_nbytes;
    int32_t slab_dtype;     /* rlxq_st_dtype of scales (and biases)            */
} rlxq_mlx_packed;
/* *out is set even when the return is an error (for rlxq_mlx_last_error). */
int rlxq_mlx_open(const char* path, rlxq_mlx** out);
void rlxq_mlx_close(rlxq_mlx* h);
const char* rlxq_mlx_last_error(const rlxq_mlx* h);
/* The checkpoint-wide quantization block (bits = group_size = 0 and
 * RLXQ_MLX_MODE_NONE when there is none). */
int rlxq_mlx_quantization(const rlxq_mlx* h, int* bits, int* group_size,
                          int* mode);
int64_t rlxq_mlx_tensor_count(const rlxq_mlx* h);
int64_t rlxq_mlx_find_tensor(const rlxq_mlx* h, const char* name);
int rlxq_mlx_tensor_info(const rlxq_mlx* h, int64_t i, rlxq_mlx_tensor* info);
/* take_packed_mlx(key): the Linear `key` (tensors key.weight, key.scales,
 * key.biases) under the quantization that applies to it (a per-layer entry
 * of the block, else the block itself).  A Linear stored dense, switched off
 * by a `false` entry, or packed in a form these kernels do not read (bits
 * other than 4 and 8, group sizes other than 32/64/128, MXFP4 other than
 * 4-bit group 32) gives scheme 0 and RLXQ_OK and is not taken (the
 * reference's Ok(None)); a second take is RLXQ_E_TAKEN. */
int rlxq_mlx_take_packed(rlxq_mlx* h, const char* key, rlxq_mlx_packed* out);
/* A tensor's bytes as stored, into host memory of cap bytes (pread). */
int rlxq_mlx_read(rlxq_mlx* h, const char* name, void* dst, size_t cap);
/* An F32 / F16 / BF16 tensor as f32, into count floats (F16 scale slabs:
 * the kernels take F32 or BF16 slabs). */
int rlxq_mlx_read_f32(rlxq_mlx* h, const char* name, float* dst, size_t count);
/* A tensor's bytes as stored, into device memory of cap bytes (pread into two
 * 32 MiB pinned staging buffers copied on `stream`, as rlxq_gguf_upload). */
int rlxq_mlx_upload(rlxq_mlx* h, const char* name, void* dst, size_t cap,
                    void* stream);

#ifdef __cplusplus
}
#endif
#endif /* RLXQ_H */
