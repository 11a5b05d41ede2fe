/*
 * thq_oracle.h — CPU oracle for the GGUF block-quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * kernels are compared against; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product library (libthq)
 * never links, loads or calls it.
 *
 * What it restates.  The arithmetic of the reference's GGUF branch lives in
 * the crates.io dependency candle-core 0.11.0 (pinned at
 * engine/Cargo.lock:253-256, engine/Cargo.toml:23), reached from
 * engine/src/model.rs:551-562 (quantized_qwen3 / qwen2 / llama -> QMatMul).
 * candle-core is not vendored in the reference tree, so every candle item
 * below is restated from candle's published k_quants.rs / utils.rs (which
 * follow GGML's ggml-quants.c) and is marked [ext].  The in-tree anchors
 * are the argmax tie rule (engine/src/engine.rs:1891-1898, tests
 * :3086-3128) and the gate/up epilogue (engine/src/quant_kernel.rs:2922-2926,
 * engine/src/qwen35.rs:7002-7007).
 *
 * Pinning (how each function is checked, in tests/test_oracle.py):
 *   f16 / bf16 conversions      exhaustive round trips, IEEE special cases
 *   Q8_0 quantize / dequant     closed-form KATs (exact-in-f16 scales), error bound
 *   Q4_K dequant                hand-built superblock KATs, scale/min pack round trip
 *   Q4_K quantize               grid-exact sub-blocks (x = s*l - m, s and m powers
 *                               of two: levels and (s, m) exact); the largest
 *                               stored 6-bit scale / min is 63; literal bytes
 *                               and (scale, min, levels) from an independent
 *                               float32 trace of the published algorithm
 *                               (tests/golden/make_quant_vectors.py), drawn so
 *                               that nmax 14, ntry 4 / 6 / 1 or 64/max fail
 *   Q8_K quantize               KAT at iscale = 1 (x.5 ties round away from
 *                               zero, clamp to 127, first of equal |x|) and
 *                               literal blocks from the same trace
 *   vec_dot Q8_0xQ8_0 / Q4_KxQ8_K  exact integer brute force on small inputs;
 *                               f32 accumulation order parity unpinned
 *   matmul DEQUANT_F32          brute force f64 on tiny shapes
 *   argmax                      the reference's own tie vectors
 *   gate/up SiLU epilogue       the reference test's closed form
 *   Q6_K dequant                hand-built blocks with literal expected floats,
 *                               every 6-bit code and every scale byte, and an
 *                               independent numpy formula on random bytes
 *   MLX affine dequant          an independent numpy formula with correct
 *                               rounding (equal wherever half's truncation of
 *                               the low f64 bits cannot matter); the half
 *                               truncation rule itself by KATs of its
 *                               published algorithm
 *   QLin::tiled                 the q4woff / q4sb address formulas
 */
#ifndef THQ_ORACLE_H
#define THQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML block sizes / byte sizes */
#define OQK8_0 32
#define OQK_K 256
#define O_Q8_0_BYTES 34  /* f16 d + 32 x i8 */
#define O_Q4_K_BYTES 144 /* f16 d + f16 dmin + 12 B scales + 128 B nibbles */
#define O_Q8_K_BYTES 292 /* f32 d + 256 x i8 + 16 x i16 bsums */
#define O_Q6_K_BYTES 210 /* u8 ql[128] + u8 qh[64] + i8 scales[16] + f16 d */

/* GGML type ids (the values GGUF files carry) */
#define O_TYPE_Q8_0 8
#define O_TYPE_Q4_K 12
#define O_TYPE_Q6_K 14

/* ---- scalar conversions ---- */
float o_f16_to_f32(uint16_t h);
uint16_t o_f32_to_f16(float f);   /* round to nearest even, like half::f16::from_f32 */
float o_bf16_to_f32(uint16_t h);
uint16_t o_f32_to_bf16(float f);  /* round to nearest even, like half::bf16::from_f32 */
float o_bf16_round(float f);      /* f32 -> bf16 -> f32 */

/* ---- seeded synthetic inputs: splitmix64 -> Box-Muller (f64) -> f32 ---- */
void o_randn(uint64_t seed, uint64_t stream, float sigma, float* out, size_t n);

/* ---- block formats ---- */
size_t o_row_bytes(int type, int64_t k);
void o_quantize_q8_0(const float* x, uint8_t* blocks, int64_t k);
void o_dequantize_q8_0(const uint8_t* blocks, float* y, int64_t k);
void o_quantize_q4_k(const float* x, uint8_t* blocks, int64_t k);
void o_dequantize_q4_k(const uint8_t* blocks, float* y, int64_t k);
void o_quantize_q8_k(const float* x, uint8_t* blocks, int64_t k);
void o_dequantize_q6_k(const uint8_t* blocks, float* y, int64_t k);
void o_get_scale_min_k4(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
/* levels (nullable): the n levels of the last refinement pass (0 when max == min) */
void o_make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* scale, float* min_out, uint8_t* levels);

/* whole matrices [n rows][k] */
int o_quantize(int type, const float* w, int64_t n, int64_t k, uint8_t* out);
int o_dequantize(int type, const uint8_t* blocks, int64_t n, int64_t k, float* out);

/* ---- dot products (candle vec_dot_unopt order) ---- */
float o_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w_blocks, const uint8_t* x_blocks);
float o_vec_dot_q4_k_q8_k(int64_t k, const uint8_t* w_blocks, const uint8_t* x_blocks);

/* ---- matmul y[m][n] = x[m][k] . W[n][k]^T ----
 * mode 0 = DEQUANT_F32: dequantize W exactly, accumulate in f64, round to f32
 *          (candle's CANDLE_DEQUANTIZE_ALL semantics, with a better accumulator)
 * mode 1 = Q8ACT: candle's default CPU path (quantize x rows to the weight's
 *          VecDotType, integer block dots, f32 block scaling)
 * threads: 0 = all OpenMP threads */
int o_matmul(int type, int mode, const uint8_t* w, int64_t n, int64_t k, const float* x, int64_t m,
             float* y, int threads);

/* ---- epilogues / consumers ---- */
/* y_gu[m][2h] (gate rows 0..h-1, up rows h..2h-1)  ->  out[m][h] bf16 bits */
void o_gate_up_silu(const float* y_gu, int64_t m, int64_t h, uint16_t* out_bf16);
/* strict '>' scan from (0, -inf): lowest index among equal maxima, NaN never wins */
uint32_t o_argmax(const float* v, int64_t n);
void o_argmax_rows(const float* v, int64_t m, int64_t n, uint32_t* idx);

/* ---- MLX affine 4-bit (affine_oracle.c) ---- */
uint16_t o_bf16_from_f64_half(double v); /* [ext] half 2.7.1 bf16::from_f64 */
void o_affine_dequant_bf16(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, uint16_t* out);
void o_affine_dequant_f32(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, float* out);
void o_affine_matmul(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, const float* x, int64_t m,
                     float* y);
void o_affine_tile(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, uint32_t* wq_t, uint16_t* sb_t);

/* ---- CPU baseline: AVX2 + OpenMP Q8ACT matmul (falls back to scalar) ---- */
int o_baseline_matmul(int type, const uint8_t* w, int64_t n, int64_t k, const float* x, int64_t m,
                      float* y, int threads);
int o_baseline_has_avx2(void);
int o_max_threads(void);

/* Per-row top-k by (key desc, id asc), key(NaN) = -inf, key(-0) = +0
 * (engine/src/sample_kernel.rs:163-169, 326-347); slots past n: (-inf, 0xFFFFFFFF). */
void o_topk_rows(const float* v, int64_t m, int64_t n, int k, float* vals, uint32_t* idx);

#ifdef __cplusplus
}
#endif
#endif
