// thq_kernels.hpp — host-side launchers of the gfx950 kernels (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace thq {

// A weight as the kernels see it (device layouts; download restores GGUF bytes).
//   Q8_0 (qtype 8):  q   = i8 tile plane, aux = f16 scale tile plane
//                    (32-row tiles: thq_dev.hpp, q8t_q / q8t_d)
//   MLX affine 4-bit (qtype 13): q = the same row-quad plane with affine
//                    headers (thq_dev.hpp, aff_scale); K may be padded to
//                    whole superblocks (zero groups)
//   Q6_K (qtype 14): q   = QL, QH, SC, D planes (thq_dev.hpp, q6k_layout)
//   Q4_K (qtype 12): q   = row-quad plane, ceil(N/4) groups of 4 x K/256 x
//                          144 B (layout in thq_dev.hpp, q4k_group); padding
//                          rows are zero
//                    aux = unused
// Fused greedy-argmax epilogue (LM head without logits in HBM): a decode
// kernel given `v` writes, per activation row m and output tile b, the tile's
// (max, index) under the argmax tie rule to v[m*ld + b], i[m*ld + b] instead
// of storing y; the launcher reports the tile count in nb (0: this path has
// no fused epilogue, nothing was launched).
struct AmaxOut {
    float* v = nullptr;
    uint32_t* i = nullptr;
    int64_t ld = 0;
    int64_t nb = 0;
};

struct WeightView {
    int qtype;
    int64_t N, K;
    const uint8_t* q;
    const uint8_t* aux;
};

struct GemmPlan {
    int bm = 64;
    int64_t tiles_n = 0, tiles_m = 0;
    int splits = 1, kps = 0;
    size_t workspace_bytes = 0;
};

// weights
// Q8_0: n rows of nb = K / 32 blocks, into / out of the tile planes (thq_dev.hpp, q8t_q / q8t_d)
hipError_t launch_repack_q8_0(const uint8_t* raw, int8_t* qs, uint16_t* d, int64_t n, int64_t nb, hipStream_t s);
hipError_t launch_quantize_q8_0(const float* w, int8_t* qs, uint16_t* d, int64_t n, int64_t nb, hipStream_t s);
hipError_t launch_q8_0_copy_rows(const int8_t* sq, const uint16_t* sd, int64_t nsrc, int8_t* dq, uint16_t* dd,
                                 int64_t row0, int64_t nb, hipStream_t s);
hipError_t launch_quantize_q4k(const float* w, uint8_t* dst, int64_t n, int nsb, hipStream_t s);
// GGUF Q4_K blocks -> row-quad plane (rows dst_row0 ..)
hipError_t launch_repack_q4k(const uint8_t* gguf, uint8_t* dst, int64_t n, int nsb, hipStream_t s);
// copy rows between row-quad planes (weight fusion)
hipError_t launch_q4k_copy_rows(const uint8_t* src, int64_t n, uint8_t* dst, int64_t dst_row0, int nsb, hipStream_t s);
// dequantization to f32 (bf16 = false) or bf16
hipError_t launch_dequant_q8_0(const int8_t* qs, const uint16_t* d, void* out, bool bf16, int64_t n, int64_t nb,
                               hipStream_t s);
hipError_t launch_dequant_q4k(const uint8_t* src, void* out, bool bf16, int64_t n, int nsb, hipStream_t s);
// Q6_K (qtype 14): GGUF blocks -> planes (thq_dev.hpp, q6k_layout), dequantization
hipError_t launch_repack_q6k(const uint8_t* gguf, uint8_t* dst, int64_t n, int nsb, hipStream_t s);
hipError_t launch_dequant_q6k(const uint8_t* src, void* out, bool bf16, int64_t n, int nsb, hipStream_t s);
// MLX affine 4-bit (qtype 13): QLin arrays -> row-quad plane (K padded to whole
// superblocks), and its dequantization (bf16: the reference's f64 rounding)
hipError_t launch_repack_affine(const uint32_t* wq, const uint16_t* sb, uint8_t* dst, int64_t n, int K, int gs,
                                bool tiled, hipStream_t s);
hipError_t launch_dequant_affine(const uint8_t* src, void* out, bool bf16, int64_t n, int K, hipStream_t s);

// decode GEMV (M = 1); gu = fused gate/up over a [gate; up] weight
bool gemv1_supported(int qtype, int K, bool gu, int64_t n_rows);
// Q4_K / MLX affine, bf16 rows (16-B aligned), K % 256 == 0: 2 <= M <= 4 for K <= 4096, M = 2 for K <= 16384
bool gemv_rows_supported(int qtype, int M, int K, bool gu, int64_t n_rows);
hipError_t launch_gemv_rows(const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M, int64_t nout,
                            int64_t up_off, hipStream_t s);
// Q6_K M = 1 with bf16 x (K % 256 == 0, K <= 16384), k_q6k.hip
hipError_t launch_gemv1_q6k(const WeightView& w, const void* x, void* y, bool yf32, bool gu, int64_t nout,
                            int64_t up_off, hipStream_t s, AmaxOut* am = nullptr);
hipError_t launch_gemv1(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int64_t nout,
                        int64_t up_off, hipStream_t s, AmaxOut* am = nullptr);
// decode GEMV on MFMA: 1 <= M <= 8 bf16 activation rows, exact weights
struct GemvPlan {
    int waves = 0, cpw = 0, splits = 0;  // waves per block, 256-wide chunks per wave, K splits
    size_t workspace_bytes = 0;          // split partials (f32 [splits][M][N])
};
GemvPlan plan_gemv_mfma(int qtype, int64_t M, int64_t N_rows, int64_t K, bool gu);  // waves == 0: unsupported
// the kernel instance a plan launches (E live accumulator rows per lane, NX
// staged activation chunks per thread); E == 0: none
struct GemvInstance {
    int E = 0, NX = 0;
};
GemvInstance gemv_mfma_instance(int qtype, int M, const GemvPlan& p);
// the kernel's LDS staging limits (bf16 elements / float sums)
struct GemvLimits {
    int xs_elems, xs_pad_elems, kb_max, kb_max_e8, mmax, max_waves;
    int sums_rows_e4, sums_rows_e8, sums_cols_e4, sums_cols_e8;
};
GemvLimits gemv_mfma_limits();
hipError_t launch_gemv_mfma(const GemvPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M,
                            int64_t nout, int64_t up_off, float* ws, hipStream_t s, AmaxOut* am = nullptr);
// exact-weight GEMV for 1 <= M <= 64 bf16 rows (16-B aligned), K % 256 == 0,
// Q8_0 / Q4_K / MLX affine / Q6_K, plain or gate/up (k_gemv_wide.hip)
struct WidePlan {
    int splits = 0, cps = 0;      // K splits, 256-wide chunks per split (splits == 0: unsupported)
    size_t workspace_bytes = 0;   // split partials (f32 [splits][M][N])
};
WidePlan plan_gemv_wide(int qtype, int64_t M, int64_t N, int64_t K, int cus);
hipError_t launch_gemv_wide(const WidePlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu,
                            int M, int64_t nout, int64_t up_off, float* ws, hipStream_t s, AmaxOut* am = nullptr);
// prefill / verify GEMM with rounded weights for Q4_K / MLX affine on the
// row-quad plane (k_gemm_mid.hip): bf16 rows (16-B aligned), K % 256 == 0,
// plain or gate/up; activation rows in groups of 32 mh (grid.z)
struct MidPlan {
    int mh = 0, nt = 1, nw = 4, groups = 0;  // 32-row halves per group (2 or 4; 0: unsupported), column tiles per wave, waves per block, groups
    int splits = 0, cps = 0;      // K splits, 256-wide chunks per split
    size_t workspace_bytes = 0;   // split partials (f32 [splits][M][N])
};
MidPlan plan_gemm_mid(int qtype, int64_t M, int64_t N, int64_t K, bool gu, int cus);
hipError_t launch_gemm_mid(const MidPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M,
                           int64_t nout, int64_t up_off, float* ws, hipStream_t s);
// Q4_K / MLX affine tile plane (thq_dev.hpp, q4t_record), k_gemv_tile.hip:
// its size, its construction from the row-quad plane, and the 3..8-row
// decode GEMV over it (bf16 rows, 16-B aligned; plain or gate/up)
size_t tile_plane_bytes(int64_t n, int64_t k);
hipError_t launch_repack_q4t(const uint8_t* rowquad, uint8_t* tiles, int64_t n, int64_t k, hipStream_t s);
struct TilePlan {
    int kw = 0, splits = 0;       // waves per block (0: unsupported), K splits
    size_t workspace_bytes = 0;   // split partials (f32 [splits][M][N])
};
// gu: fused gate/up over a [gate; up] weight (N a multiple of 64)
TilePlan plan_gemv_tile(int64_t M, int64_t N, int64_t K, bool gu, int cus);
// cnt: null, or ceil(nout / 32) u32 arrival counters that are zero (and stay
// zero after the launch) for the last-block reduction of K splits;
// without them a split plan runs k_split_reduce after the kernel
hipError_t launch_gemv_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* x, void* y,
                            bool yf32, bool gu, int M, float* ws, uint32_t* cnt, hipStream_t s);
// THQ_MODE_Q8ACT over the Q4_K tile plane (1..8 rows): the Q8_K planes xq
// [M][K] i8, xd [M][K/256] f32, xb [M][K/32] i16 against the weight with
// int8 MFMAs; plan, partials and counters as launch_gemv_tile
hipError_t launch_q8act_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const int8_t* xq,
                             const float* xd, const int16_t* xb, void* y, bool yf32, bool gu, int M, float* ws,
                             uint32_t* cnt, hipStream_t s);
// sum split partials P[s][M][ldp] in split order, then the epilogue
hipError_t launch_split_reduce(const float* P, void* y, bool yf32, bool gu, int M, int64_t nout, int64_t up_off,
                               int64_t ldp, int splits, hipStream_t s);
// prefill GEMM with the Q4_K / MLX affine weight dequantized into LDS
// (k_gemm_fq.hip): geometry (block tile), grid and K splits of a call
struct FqPlan {
    int geom = 1;  // 1: 256 x 256 (gate/up: always), 2: 128 x 256, 3: 512 x 192
    int tiles_m = 0, tiles_n = 0;
    int kps = 0, splits = 1;  // 32-wide K steps per split
    size_t workspace_bytes = 0;  // split partials, f32 [splits][M][N rows]
};
bool gemm_fq_supported(int64_t M, int64_t N_rows, int64_t K, bool gu);
FqPlan plan_gemm_fq(int64_t M, int64_t N_rows, int64_t K, bool gu, int cus);
hipError_t launch_gemm_fq(const FqPlan& p, bool aff, const uint8_t* wq, const void* x, void* y, bool yf32, bool gu,
                          int M, int64_t N_rows, int K, float* ws, hipStream_t s);
// mid-M prefill GEMM with the Q4_K / MLX affine weight dequantized in
// registers into MFMA operands (k_gemm_rq.hip): block tile, grid and K splits
struct RqPlan {
    int bm = 256;  // block rows of M (128 or 256); 128 weight rows per block
    int tiles_m = 0, tiles_n = 0;
    int whole = 0;            // tiles computed over all of K (the first blocks); the rest are split
    int kps = 0, splits = 1;  // 64-wide K steps per split
    int64_t counters = 0;     // arrival counters the split reduction needs (one per split tile)
    size_t workspace_bytes = 0;  // split partials, f32, one BM x 128 tile per (tile, split)
};
bool gemm_rq_supported(int qtype, int64_t M, int64_t N_rows, int64_t K, bool gu);
RqPlan plan_gemm_rq(int64_t M, int64_t N_rows, int64_t K, bool gu, int cus);
hipError_t launch_gemm_rq(const RqPlan& p, bool affine, const uint8_t* wq, const void* x, void* y, bool yf32, bool gu,
                          int M, int64_t N_rows, int K, float* ws, uint32_t* cnt, hipStream_t s);
// exact generic kernel, any M, scalar activation loads
hipError_t launch_generic(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int M,
                          int64_t nout, int64_t up_off, hipStream_t s);

// MFMA GEMM (bf16 activations)
// cus: compute units of the device (the split count fills whole rounds of them)
GemmPlan plan_gemm(int qtype, bool exact, int64_t M, int64_t N_rows, int64_t K, bool gu, int cus);
hipError_t launch_gemm(const GemmPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, bool exact,
                       int M, float* ws, hipStream_t s);

// bf16 x bf16 GEMM over a weight dequantized to bf16 [N][K] (k_gemm_b16.hip),
// the dequantize-then-GEMM prefill route: K % 32 == 0, x and Wb below 4 GiB
bool gemm_b16_supported(int64_t M, int64_t N, int64_t K);
int64_t gemm_b16_blocks(int64_t M, int64_t N);  // 256 x 384 output tiles
hipError_t launch_gemm_b16(const void* x, const void* wb, void* y, bool yf32, int M, int N, int K, hipStream_t s);

// THQ_MODE_Q8ACT: activation quantization + exact integer block dots
bool q8act_supported(int qtype, int64_t K);
size_t q8act_workspace_bytes(int qtype, int64_t M, int64_t K);
hipError_t launch_q8act(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int M,
                        int64_t nout, int64_t up_off, void* ws, hipStream_t s);
// THQ_MODE_Q8ACT in two steps: the activation planes (q8act_workspace_bytes,
// 256-B aligned) written once by the quantizer, then read by any number of
// dot launches over weights of the same dot type and K
hipError_t launch_q8act_prepare(int qtype, const void* x, bool xf32, int64_t M, int64_t K, void* planes,
                                hipStream_t s);
hipError_t launch_q8act_dot(const WeightView& w, const void* planes, void* y, bool yf32, bool gu, int M, int64_t nout,
                            int64_t up_off, hipStream_t s);
// the same dot over the weight's tile plane (Q4_K, 1..8 rows), and the
// quantize + tile dot in one call (the planes at `planes`, split partials at ws)
hipError_t launch_q8act_dot_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* planes,
                                 void* y, bool yf32, bool gu, int M, float* ws, uint32_t* cnt, hipStream_t s);
hipError_t launch_q8act_tiled(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* x, bool xf32,
                              void* y, bool yf32, bool gu, int M, void* planes, float* ws, uint32_t* cnt,
                              hipStream_t s);
// Q4_K gate/up over Q8_K planes that also emits the Q8_K planes of its own
// output y [M][nout] (nout % 256 == 0) into out_planes; counters: zeroed u32
// [q8act_emit_counters(M, K, nout)], zero again when the launch completes
size_t q8act_emit_counters(int64_t M, int64_t K, int64_t nout);
hipError_t launch_q8act_dot_emit(const WeightView& w, const void* planes, void* y, bool yf32, int M, int64_t nout,
                                 uint32_t* counters, void* out_planes, hipStream_t s);
// GGML blocks of the dot type (qtype 8 -> Q8_0 blocks, 12 -> Q8_K blocks)
hipError_t launch_quantize_act(int qtype, const void* x, bool xf32, int64_t M, int64_t K, void* blocks,
                               hipStream_t s);

// argmax
size_t argmax_workspace_bytes(int64_t m, int64_t n);
hipError_t launch_argmax(const float* v, int64_t m, int64_t n, uint32_t* idx, void* ws, hipStream_t s);
// reduce fused-epilogue partials v / i [m][ld] (nb per row) to idx[m]; tmp
// holds argmax_partials_tmp_bytes(m, nb)
size_t argmax_partials_tmp_bytes(int64_t m, int64_t nb);
hipError_t launch_argmax_partials(const float* v, const uint32_t* i, int64_t m, int64_t nb, int64_t ld,
                                  uint32_t* idx, void* tmp, hipStream_t s);

// exact per-row top-k (k <= 64) by (logit desc, id asc), k_topk.hip.  cnt:
// ncnt zeroed arrival counters (left zero), or null; with at least
// topk_counters(m) of them, rows of up to 64 segments of 4096 logits take
// one launch per 2048 rows
size_t topk_workspace_bytes(int64_t m, int64_t n, int k);
int64_t topk_counters(int64_t m);
hipError_t launch_topk(const float* v, int64_t m, int64_t n, int k, float* vals, uint32_t* idx, void* ws,
                       uint32_t* cnt, int64_t ncnt, hipStream_t s);

}  // namespace thq
