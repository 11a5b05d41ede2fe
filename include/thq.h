/*
 * thq.h — C ABI of the MI355X block-quantized matmul library (libthq.so).
 *
 * This is the drop-in boundary for token-horizon's quantized projection path:
 * the GGUF Q8_0 / Q4_K weight x activation GEMV/GEMM that the engine runs for
 * every Qwen-class projection, the fused gate/up MLP projection and the LM
 * head (including the speculative-decode verify step).
 *
 * Conventions
 *  - Plain C: pointers, sizes, enums.  No torch or HIP types cross the ABI;
 *    `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *  - Device pointers are marked *_dev.  Calls are stream-ordered and
 *    asynchronous unless stated otherwise.
 *  - Every function returns THQ_OK (0) or a negative error code; the message
 *    of the last failure on the calling thread is thq_last_error().  No C++
 *    exception ever crosses the ABI.
 *  - Weights are immutable after creation and may be shared by any number of
 *    concurrent calls.  A weight belongs to its device, not to the context
 *    that made it: it may be freed before or after that context.
 *  - Workspace.  Calls whose kernels need device scratch (split-K partials,
 *    quantized activation planes, argmax partials, LM-head logits without a
 *    logits buffer) take it from their context's workspace.  Calls on
 *    distinct streams are re-entrant, except that calls sharing one
 *    context's workspace must be ordered on one stream.  The workspace grows
 *    (hipMalloc, no device synchronization) the first time a larger shape
 *    arrives; the buffer it outgrew stays allocated until thq_destroy, so
 *    work already enqueued, or captured in a HIP graph, keeps valid memory.
 *    A call that grows the workspace cannot run under stream capture: warm
 *    every captured shape once beforehand.
 *  - W is [N, K] row-major (row n = output feature n), exactly the GGUF
 *    tensor layout QTensor::data() returns.  y[m, n] = sum_k x[m, k] * W[n, k].
 */
#ifndef THQ_H
#define THQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- enums ---- */

/* GGML type ids, as stored in GGUF files.
 * Replaces candle-core's GgmlDType (Q8_0, Q4K) that QTensor::dtype() returns
 * on the path engine/src/model.rs:551-562 -> quantized_qwen3::ModelWeights. */
typedef enum thq_dtype {
    THQ_Q8_0 = 8,  /* 32 weights / 34 B: f16 d, i8 qs[32]                        */
    THQ_Q4_K = 12, /* 256 weights / 144 B: f16 d, f16 dmin, u8 scales[12], u8 qs[128] */
    THQ_Q6_K = 14, /* 256 weights / 210 B: u8 ql[128], u8 qh[64], i8 scales[16], f16 d;
                      w = d * scale[j/16] * (6-bit code - 32) ([ext] candle-core 0.11
                      BlockQ6K::to_float); the type a Q4_K_M file keeps its output
                      head and part of ffn_down / attn_v in (read by the loader at
                      engine/src/model.rs:526-562)                               */
    THQ_Q8_K = 15, /* 256 activations / 292 B: f32 d, i8 qs[256], i16 bsums[16]
                      (dot type of Q4_K; thq_quantize_act only)                   */
    THQ_MLX_Q4 = 100 /* MLX affine 4-bit, the engine's own QLin format (not a GGML id):
                        u32 wq [N][K/8], 8 nibbles per word LSB first; bf16 sb
                        [N][2*K/gs], each row's K/gs scales then its K/gs biases;
                        w[n][k] = q * scale[n][k/gs] + bias[n][k/gs]             */
} thq_dtype;

/* activation / output element types */
typedef enum thq_act {
    THQ_ACT_F32 = 0,
    THQ_ACT_BF16 = 1
} thq_act;

/* thq_matmul flags */
#define THQ_MODE_DEQUANT_F32 0u /* y = x . dequant(W)^T, f32 accumulation (default)  */
#define THQ_MODE_Q8ACT 0x1u     /* candle's default CPU semantics: x rows quantized to
                                   Q8_0 (Q8_0 W) or Q8_K (Q4_K W), exact integer
                                   block dots, f32 block scaling                     */
#define THQ_MODE_EXACT_W 0x10u  /* never round dequantized weights to bf16 on MFMA   */
#define THQ_MODE_ARGMAX_FUSED 0x20u /* thq_matmul_argmax with logits_dev NULL only: fuse
                                       the argmax into the decode kernels' epilogue */

/* error codes */
#define THQ_OK 0
#define THQ_EINVAL (-1)       /* null pointer, bad enum, bad flag            */
#define THQ_ESHAPE (-2)       /* K not a multiple of the block, dims mismatch */
#define THQ_EDTYPE (-3)       /* unsupported dtype combination                */
#define THQ_EALIGN (-4)       /* device pointer alignment the call requires   */
#define THQ_EHIP (-5)         /* HIP runtime error                            */
#define THQ_ENOMEM (-6)       /* device allocation failed                     */
#define THQ_EIO (-7)          /* a file cannot be opened or mapped            */
#define THQ_EFORMAT (-8)      /* malformed or unsupported GGUF file           */
#define THQ_ENOTFOUND (-9)    /* no such GGUF tensor or metadata key          */

typedef struct thq_ctx thq_ctx;
typedef struct thq_weight thq_weight;

/* ---- context ---- */

/* One context per device: owns the device's workspace and kernel state.
 * Replaces the process-global pipeline/OnceLock state of the reference's ops
 * (engine/src/quant_kernel.rs:2980-2987, 3008-3038) and candle's Device. */
int thq_init(int device, thq_ctx** out);
void thq_destroy(thq_ctx* ctx);

/* Message of the last failure on the calling thread ("" if none). */
const char* thq_last_error(void);

/* Library version string. */
const char* thq_version(void);

/* ---- weights ---- */

/* Copy GGUF block bytes (host memory, [N][K/bs] blocks row-major, exactly
 * QTensor::data()) to the device.  The library may repack on device; the
 * handle owns its device memory.  Synchronous.  Every weight (any creation
 * call) has N >= 1, K a positive multiple of the block size, K <= 2^30,
 * N <= 2^40 and at most 2^46 packed bytes; THQ_ESHAPE otherwise.
 * Replaces candle's QTensor::new / QMatMul::from_arc
 * (reached from engine/src/model.rs:551-562). */
int thq_weight_upload(thq_ctx* ctx, thq_dtype dtype, const void* host_blocks, int64_t n, int64_t k,
                      thq_weight** out);

/* As thq_weight_upload, from GGUF block bytes already in device memory
 * (16-byte aligned for Q4_K, 2-byte aligned for Q8_0 and Q6_K). */
int thq_weight_from_device(thq_ctx* ctx, thq_dtype dtype, const void* dev_blocks, int64_t n, int64_t k,
                           void* stream, thq_weight** out);

/* Quantize an f32 [N, K] device matrix to `dtype` on the device, with the
 * same rounding rules as candle's CPU quantizer (BlockQ8_0::from_float,
 * BlockQ4K::from_float).  Replaces QTensor::quantize. */
int thq_quantize(thq_ctx* ctx, thq_dtype dtype, const float* w_dev, int64_t n, int64_t k, void* stream,
                 thq_weight** out);

/* Row-concatenate weights of one dtype and K: QKV = [q; k; v], gate|up =
 * [gate; up].  Replaces QLin fusion (engine/src/qwen35.rs:1581-1621 fuse_lins). */
int thq_weight_fuse(thq_ctx* ctx, const thq_weight* const* parts, int nparts, thq_weight** out);

/* Give a Q4_K or MLX affine weight a second, tile-major copy (32-row tiles,
 * built on the device from the weight's own planes; synchronous).  With it,
 * thq_matmul runs 3..8 bf16 activation rows of a plain projection on the
 * tile-plane decode GEMV (exact weights, whole-line loads) instead of the
 * row-layout kernels, and so does thq_gate_up_silu on a fused [gate; up]
 * weight whose halves are whole 32-row tiles.  THQ_MODE_Q8ACT calls and
 * thq_matmul_q8act / thq_gate_up_silu_q8act on a Q4_K weight with a tile
 * plane run 2..8 rows on it with int8 matrix-core dots (same results to the
 * f32 summation order).  Every other call is unchanged.  It doubles the
 * weight's device memory, which thq_weight_free releases.  Idempotent.  Call
 * it before the weight is shared with other threads or used by work in
 * flight (it adds to the weight handle).  A fused weight does not inherit
 * its parts' tile planes.  THQ_EDTYPE for other dtypes.  Replaces the
 * engine's tiled weight repack for its few-row kernels (QLin::tiled,
 * engine/src/qwen35.rs:629-697). */
int thq_weight_add_tiles(thq_ctx* ctx, thq_weight* w);

void thq_weight_free(thq_weight* w);

/* Shape / dtype / GGUF byte size of a weight. */
int thq_weight_info(const thq_weight* w, thq_dtype* dtype, int64_t* n, int64_t* k, size_t* gguf_bytes);

/* Copy the GGUF block bytes back to host memory (QTensor::data()).  Synchronous. */
int thq_weight_download(const thq_weight* w, void* host_blocks);

/* MLX affine 4-bit weights (THQ_MLX_Q4), the engine's QLin
 * (engine/src/qwen35.rs:311-319: wq U32 [out, in/8], sb BF16 [out, 2*ng]).
 * `tiled` = 0: row-major arrays as QLin::new takes them; `tiled` = 1: the
 * QLin::tiled layout (qwen35.rs:629-697; word / scale addresses q4woff / q4sb,
 * engine/src/quant_kernel.rs:1085-1101): wq [ceil(N/256)][K/64][256][8],
 * scales [(tile*ng + g)*256 + col] and biases after all ceil(N/256)*ng*256
 * scales, rows padded to 256.  K must be a multiple of 64, gs a multiple of
 * 64 dividing K (64 for tiled).  Synchronous.  Replaces the QLin constructors
 * (Weights::get_lin, qwen35.rs:249-300) and QLin::tiled. */
int thq_affine_upload(thq_ctx* ctx, const uint32_t* wq_host, const uint16_t* sb_host, int64_t n, int64_t k, int gs,
                      int tiled, thq_weight** out);
int thq_affine_from_device(thq_ctx* ctx, const uint32_t* wq_dev, const uint16_t* sb_dev, int64_t n, int64_t k, int gs,
                           int tiled, void* stream, thq_weight** out);
/* The row-major QLin arrays back (wq [N][K/8], sb [N][2*K/gs]).  Synchronous. */
int thq_affine_download(const thq_weight* w, uint32_t* wq_host, uint16_t* sb_host);

/* ---- compute ---- */

/* Exact f32 dequantization, out_dev [N, K] (QTensor::dequantize). Bit-exact
 * with candle's BlockQ8_0/BlockQ4K/BlockQ6K::to_float.  MLX affine: q*scale + bias
 * rounded once to f32. */
int thq_dequantize(thq_ctx* ctx, const thq_weight* w, float* out_dev, void* stream);

/* bf16 dequantization, out_dev [N, K] bf16 bits, 16-byte aligned.  MLX
 * affine: bit-exact with dequant_affine (engine/src/qwen35.rs:110-134:
 * bf16::from_f64(q * scale + bias)) and AffineDequant's W -> bf16 scratch
 * (engine/src/quant_kernel.rs:1035-1040); GGUF types: the f32 values of
 * thq_dequantize rounded to nearest even. */
int thq_dequantize_bf16(thq_ctx* ctx, const thq_weight* w, uint16_t* out_dev, void* stream);

/* Quantize activation rows x[M, K] (f32 or bf16, 16-byte aligned) to GGML
 * blocks of `dot_type`: THQ_Q8_0 (34-B blocks, 2-byte aligned blocks_dev) or
 * THQ_Q8_K (292-B blocks, 4-byte aligned), M * K/bs blocks row-major.
 * Bit-identical to [ext] candle-core 0.11 BlockQ8_0::from_float /
 * BlockQ8K::from_float, the first step of k_quants::matmul that candle's
 * QMatMul::forward runs for quantized weights (and the step THQ_MODE_Q8ACT
 * runs inside thq_matmul).  bf16 x is widened to f32 exactly first. */
int thq_quantize_act(thq_ctx* ctx, thq_dtype dot_type, const void* x_dev, thq_act x_type, int64_t m, int64_t k,
                     void* blocks_dev, void* stream);

/* Producer-side activation operand for THQ_MODE_Q8ACT ("presum": the
 * producer emits what every consumer would otherwise recompute; the engine's
 * presum blocks, engine/src/quant_kernel.rs:265-321).  candle's default
 * QMatMul::forward quantizes its input once per call, so projections that
 * share an input (q / k / v, gate / up) quantize the same rows again.  Here
 * thq_q8act_prepare quantizes x [M, K] once into an opaque device buffer of
 * thq_q8act_bytes(dot_type, m, k) bytes (256-byte aligned), and
 * thq_matmul_q8act / thq_gate_up_silu_q8act consume it for any number of
 * weights whose dot type it is (THQ_Q8_0 for Q8_0 weights, THQ_Q8_K for
 * Q4_K) and whose K is k.  Results are bit-identical to thq_matmul /
 * thq_gate_up_silu with THQ_MODE_Q8ACT on the same x.  Returns 0 for an
 * unsupported dot type. */
size_t thq_q8act_bytes(thq_dtype dot_type, int64_t m, int64_t k);
int thq_q8act_prepare(thq_ctx* ctx, thq_dtype dot_type, const void* x_dev, thq_act x_type, int64_t m, int64_t k,
                      void* buf_dev, void* stream);
int thq_matmul_q8act(thq_ctx* ctx, const thq_weight* w, thq_dtype dot_type, const void* buf_dev, int64_t m,
                     int64_t k, void* y_dev, thq_act y_type, void* stream);
int thq_gate_up_silu_q8act(thq_ctx* ctx, const thq_weight* fused, thq_dtype dot_type, const void* buf_dev,
                           int64_t m, int64_t k, void* y_dev, thq_act y_type, void* stream);

/* thq_gate_up_silu_q8act that also emits the next projection's operand: the
 * gate/up producer writes, besides y [M, H], the Q8_K activation buffer of y
 * into next_buf_dev (thq_q8act_bytes(THQ_Q8_K, m, H) bytes, 256-byte
 * aligned), byte-identical to thq_q8act_prepare(THQ_Q8_K, y, ...), so the
 * down projection (thq_matmul_q8act with K = H) needs no quantize launch.
 * The reference's gate/up tile likewise emits down's presum
 * (engine/src/quant_kernel.rs:3205-3207; producers :265-274).  Q4_K
 * [gate; up] weights with H a multiple of 256; y_dev 16-byte aligned.  The
 * epilogue counts arriving blocks per 256-wide segment in a small counter
 * buffer the context owns (allocated and zeroed on the first call of a
 * larger shape; each launch leaves it zero), so such calls on one context
 * must be ordered on one stream.  A weight with a tile plane
 * (thq_weight_add_tiles) at 2..8 rows instead runs its int8 tile kernel and
 * then quantizes y in a second launch: the same bytes, faster there. */
int thq_gate_up_silu_q8act_emit(thq_ctx* ctx, const thq_weight* fused, thq_dtype dot_type, const void* buf_dev,
                                int64_t m, int64_t k, void* y_dev, thq_act y_type, void* next_buf_dev,
                                void* stream);

/* y[M, N] = x[M, K] . W^T with f32 accumulation.
 * Replaces QMatMul::forward ([ext] candle-core 0.11 quantized/mod.rs, called
 * for every projection by quantized_qwen3) and the engine's routed projection
 * QLin::linear_ps (engine/src/qwen35.rs:398-617).  Routes by M internally:
 *   M == 1     decode GEMV (exact dequantized weights)
 *   M = 2..16  bf16 x with K a multiple of 256: matrix-core decode GEMV
 *              (exact weights); Q4_K / MLX affine at M = 2..4 and K <= 4096
 *              use a VALU row GEMV (exact weights) instead, and a weight
 *              with a tile plane (thq_weight_add_tiles) runs 3..8 rows on
 *              the tile-plane GEMV (exact weights)
 *   M = 17..64 bf16 x with K a multiple of 256: for Q8_0, under
 *              THQ_MODE_EXACT_W, or with >= 65536 outputs (the verify LM
 *              head), a wide matrix-core GEMV that reads the weights once
 *              for all rows (exact weights)
 *   larger M   (and the other bf16 shapes with K a multiple of 64) MFMA GEMM;
 *              weights are rounded to bf16 on its tile unless THQ_MODE_EXACT_W
 *              (Q8_0, Q4_K, MLX affine: an exact tile, (128 + q) through the
 *              MFMA and each 32-wide block's scale and offset in f32).
 *              From M = 1024, where its tiles fill the GPU, a plain
 *              projection instead dequantizes W to bf16 once into the
 *              workspace (N * K * 2 bytes, the same rounded weights) and
 *              runs a bf16 MFMA GEMM on it, the engine's "dequant + bf16
 *              matmul" prefill route
 *   Q6_K under THQ_MODE_EXACT_W past 64 rows runs the exact decode GEMV in
 *   groups of 16 rows.  x f32 with M >= 2 runs an exact f32 path, and so do
 *   the remaining shapes.
 * THQ_MODE_Q8ACT instead reproduces candle's default CPU k_quants::matmul:
 * x rows are quantized as thq_quantize_act does (into the context
 * workspace), every block dot is exact in integers and scaled in f32; only
 * the f32 summation order over blocks differs from candle's (2..8 rows of
 * a Q4_K weight with a tile plane take int8 matrix-core dots over it).  Any
 * M; x must be 16-byte aligned (THQ_EALIGN otherwise).
 * Inputs: x_dev [M, K] of x_type, y_dev [M, N] of y_type, both contiguous.
 * M == 0 is a no-op.  Errors: THQ_ESHAPE for K mismatch, THQ_EINVAL for
 * null pointers. */
int thq_matmul(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m, void* y_dev,
               thq_act y_type, uint32_t flags, void* stream);

/* thq_matmul without any allocation, for callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it).  No counterpart in the reference.  Same arguments, routing, kernels
 * and results as thq_matmul; the scratch those kernels need (split-K
 * partials, THQ_MODE_Q8ACT activation planes) is a static device array of
 * thq_noalloc_scratch_bytes() bytes (64 MiB) that each device the library
 * runs on holds until the process ends, instead of the context workspace.
 * A call whose route needs more scratch than that fails with THQ_ESHAPE and
 * launches nothing.  Every call on one device shares that device's array:
 * calls that overlap on one GPU (concurrent streams, or contexts on the same
 * device) race, so order them on one stream. */
int thq_matmul_noalloc(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m,
                       void* y_dev, thq_act y_type, uint32_t flags, void* stream);
size_t thq_noalloc_scratch_bytes(void);

/* Workspace planning for callers that capture thq calls in a HIP graph (or
 * must not allocate later).  No counterpart in the reference (its Metal
 * pipelines size their scratch inside each op).  thq_call_scratch_bytes
 * plans the route one thq_matmul (gate_up = 0) or thq_gate_up_silu
 * (gate_up = 1) call of M rows would take, on the host, and returns the
 * context workspace bytes it needs (0 for routes with no scratch); no device
 * work.  thq_reserve grows the context workspace to at least
 * workspace_bytes and the context's zeroed split-K arrival counters to at
 * least `counters` entries (one per 32-row output tile of the widest
 * weight, and 32 per row of a top-k call, at most 65536), synchronously (hipMalloc, hipMemset, device synchronize); calls
 * whose needs fit then allocate nothing.  thq_workspace_bytes returns the
 * current workspace size. */
int thq_call_scratch_bytes(thq_ctx* ctx, const thq_weight* w, int64_t m, thq_act x_type, uint32_t flags,
                           int gate_up, size_t* bytes);
int thq_reserve(thq_ctx* ctx, size_t workspace_bytes, int64_t counters);
size_t thq_workspace_bytes(const thq_ctx* ctx);

/* Fused gate/up projection: `fused` = [gate; up] (2H rows).  y[M, H] =
 * bf16( silu(bf16(g)) * bf16(u) ) with silu in f32, g = x.gate^T, u = x.up^T.
 * Replaces QLin::gate_up_act_ps (engine/src/qwen35.rs:711-884) and its kernel
 * epilogue (engine/src/quant_kernel.rs:2922-2926). y_type must be BF16 or F32
 * (F32 holds the same bf16-rounded values). */
int thq_gate_up_silu(thq_ctx* ctx, const thq_weight* fused, const void* x_dev, thq_act x_type, int64_t m,
                     void* y_dev, thq_act y_type, uint32_t flags, void* stream);

/* LM head + per-row greedy argmax.  logits_dev [M, N] f32 may be NULL (the
 * logits then live in the context workspace).  With logits_dev NULL and
 * THQ_MODE_ARGMAX_FUSED, the decode kernels that have the fused epilogue
 * (M <= 8: Q8_0, Q6_K and Q4_K / MLX affine at M = 1 with K <= 4096, and
 * the M = 2..8 matrix-core path when it runs unsplit in K; M = 17..64 on the
 * wide GEMV when it runs unsplit in K) write one (max, index)
 * partial per output tile instead of logits, and one pass reduces them;
 * other shapes take the logits path.  Both give identical indices; on
 * MI355X neither is measurably faster (the logits are ~1% of the weight
 * bytes), so fusion is opt-in.  idx_dev [M] u32.  Weights are never rounded
 * (exact dequantized values), so the argmax follows the logits computed in
 * f32.  Tie rule of engine/src/engine.rs:1891-1898: lowest index among equal
 * maxima, NaN never selected, a row of -inf/NaN gives 0.
 * Replaces the verify consumer `logits.argmax(D::Minus1)`
 * (engine/src/engine.rs:1086-1087, 2438-2440) fed by the LM head
 * (engine/src/qwen35.rs:5202-5212). */
int thq_matmul_argmax(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m,
                      float* logits_dev, uint32_t* idx_dev, uint32_t flags, void* stream);

/* Exact per-row top-k of f32 v_dev [M, N] for sampled verify: vals_dev /
 * idx_dev [M, k] receive each row's k largest logits in rank order (logit
 * desc, then id asc), a NaN ranking as -inf and -0.0 as +0.0 (the values
 * written are those keys).  1 <= k <= 64; with k > N the slots past N hold
 * (-inf, 0xFFFFFFFF).  Candidates of the reference's sampled acceptance:
 * ts_topk (engine/src/sample_kernel.rs:725-796, CPU form sorted_row_dist
 * :326-347) consuming the verify logits in place (engine/src/engine.rs:
 * 2424-2436); that kernel bounds its candidate pool, this one is exact for
 * any row.  Rows of up to 64 segments of 4096 logits run in one launch per
 * 2048 rows whose last block per row merges the segments' candidates; it
 * needs 32 zeroed arrival counters per row of a launch (thq_reserve's
 * `counters`; grown on demand, so a graph-captured call reserves them first).
 * THQ_TILE_TICKET=0, longer rows or counters that cannot be allocated take a
 * second launch per merge level instead: the same results. */
int thq_topk(thq_ctx* ctx, const float* v_dev, int64_t m, int64_t n, int k, float* vals_dev, uint32_t* idx_dev,
             void* stream);

/* LM head + top-k: thq_matmul_argmax's logits (exact weights; logits_dev
 * may be NULL, the logits then live in the context workspace) followed by
 * thq_topk of every row. */
int thq_matmul_topk(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m, int k,
                    float* logits_dev, float* vals_dev, uint32_t* idx_dev, uint32_t flags, void* stream);

/* Per-row argmax of an f32 [M, N] device matrix, same tie rule
 * (candle Tensor::argmax(D::Minus1) / engine.rs greedy_argmax). */
int thq_argmax(thq_ctx* ctx, const float* v_dev, int64_t m, int64_t n, uint32_t* idx_dev, void* stream);

/* ---- GGUF files ----
 * The loader's first step (engine/src/model.rs:526-562): parse a GGUF file,
 * read metadata, hand 2-D Q8_0 / Q4_K / Q6_K tensors to the device.  Mirrors
 * [ext] candle-core 0.11 gguf_file::Content (read, metadata, tensor_infos,
 * tensor): versions 1-3, either byte order of the "GGUF" magic, strings with
 * trailing NULs dropped and invalid UTF-8 replaced by U+FFFD, dims in
 * row-major order (GGUF's ne reversed, as candle's Shape), tensor data at
 * the first multiple of general.alignment (U8/U16/U32 or non-negative
 * I8/I16/I32; else 32) after the header; a repeated key or tensor name
 * replaces the earlier one.  Host-only except thq_weight_from_gguf.  The
 * file stays memory-mapped until thq_gguf_close; returned strings and data
 * pointers live as long as the handle. */
typedef struct thq_gguf thq_gguf;

/* metadata value types (the GGUF file format's ids) */
typedef enum thq_gguf_type {
    THQ_GGUF_U8 = 0, THQ_GGUF_I8 = 1, THQ_GGUF_U16 = 2, THQ_GGUF_I16 = 3, THQ_GGUF_U32 = 4, THQ_GGUF_I32 = 5,
    THQ_GGUF_F32 = 6, THQ_GGUF_BOOL = 7, THQ_GGUF_STRING = 8, THQ_GGUF_ARRAY = 9, THQ_GGUF_U64 = 10,
    THQ_GGUF_I64 = 11, THQ_GGUF_F64 = 12
} thq_gguf_type;

/* Content::read: THQ_EIO (open / map), THQ_EFORMAT (bad magic or version,
 * truncated header, unknown value type, bool byte > 1, unknown ggml type id). */
int thq_gguf_open(const char* path, thq_gguf** out);
void thq_gguf_close(thq_gguf* g);
int thq_gguf_version(const thq_gguf* g, uint32_t* version);

/* Counts of distinct tensor names / metadata keys (-1 for a null handle). */
int64_t thq_gguf_tensor_count(const thq_gguf* g);
int64_t thq_gguf_metadata_count(const thq_gguf* g);

/* Index of tensor `name` (Content::tensor_infos lookup), -1 if absent. */
int64_t thq_gguf_find_tensor(const thq_gguf* g, const char* name);

/* TensorInfo of tensor i: name, ggml type id, n_dims (<= 4), dims[4]
 * row-major (unused entries 0), absolute file offset of its data and
 * elems / block_size * type_size bytes.  Any argument but g may be NULL. */
int thq_gguf_tensor_info(const thq_gguf* g, int64_t i, const char** name, uint32_t* ggml_type, uint32_t* n_dims,
                         uint64_t* dims, uint64_t* offset, uint64_t* nbytes);

/* The block bytes of tensor i (TensorInfo::read): a pointer into the mapping.
 * THQ_ESHAPE if elems is not a multiple of the block size, THQ_EFORMAT if
 * the bytes lie past the end of the file. */
int thq_gguf_tensor_data(const thq_gguf* g, int64_t i, const void** data, uint64_t* nbytes);

/* Key and value type of metadata entry i (the order keys first appear).
 * Keys and tensor names come back NUL-terminated (a NUL inside one ends it
 * early; GGUF writers emit none). */
int thq_gguf_metadata_key(const thq_gguf* g, int64_t i, const char** key, uint32_t* value_type);

/* Typed metadata lookups, as strict as Value::to_u32 / to_f32 / to_string:
 * THQ_ENOTFOUND if the key is absent, THQ_EDTYPE if the value has another
 * type (a U8 is not a u32).  The engine reads general.architecture,
 * {arch}.context_length and tokenizer.ggml.eos_token_id this way
 * (engine/src/model.rs:536-549). */
int thq_gguf_metadata_u32(const thq_gguf* g, const char* key, uint32_t* out);
int thq_gguf_metadata_f32(const thq_gguf* g, const char* key, float* out);
/* `len` (may be NULL) receives the byte length: a GGUF string may hold NULs */
int thq_gguf_metadata_str(const thq_gguf* g, const char* key, const char** out, uint64_t* len);
/* Element type and length of an array value (elements are not exposed). */
int thq_gguf_metadata_array(const thq_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count);

/* Upload tensor `name` as a weight: Content::tensor + QMatMul::from_qtensor
 * for the projections ModelWeights::from_gguf builds.  The tensor must be
 * 2-D [N, K] of type Q8_0, Q4_K or Q6_K (THQ_EDTYPE / THQ_ESHAPE otherwise).
 * Synchronous, as thq_weight_upload. */
int thq_weight_from_gguf(thq_ctx* ctx, const thq_gguf* g, const char* name, thq_weight** out);

#ifdef __cplusplus
}
#endif
#endif /* THQ_H */
