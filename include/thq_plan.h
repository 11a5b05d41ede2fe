/*
 * thq_plan.h — host-only planner introspection of libthq.so.
 *
 * What thq_matmul would launch for a shape, computed on the host with no
 * device work and no context: the decode GEMVs' and the GEMMs' plans, the
 * kernel instance a plan selects, and the kernels' LDS staging limits.  For
 * tests (bounds of every plan are checked off-GPU against these limits) and
 * for tuning.  No counterpart in the reference (its Metal pipelines size
 * themselves inside each op, engine/src/quant_kernel.rs:451-459, 4552-4590).
 *
 * `dtype` is a thq_dtype (THQ_Q8_0, THQ_Q4_K, THQ_Q6_K, THQ_MLX_Q4).  Each
 * returns THQ_OK, or THQ_EDTYPE / THQ_ESHAPE for arguments the planner does
 * not cover; an unsupported shape is THQ_OK with waves (or bm) = 0.
 */
#ifndef THQ_PLAN_H
#define THQ_PLAN_H

#include <stddef.h>
#include <stdint.h>

#include "thq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Decode GEMV on the matrix cores (M = 1..16 bf16 rows). */
typedef struct thq_gemv_plan_info {
    int32_t waves;            /* waves per block (0: the shape has no plan)        */
    int32_t chunks_per_wave;  /* 256-wide K chunks per wave                         */
    int32_t splits;           /* K splits (partials summed by a reduce launch)      */
    int32_t live_rows;        /* accumulator rows per lane of the instance (E)      */
    int32_t staged_per_thread;/* 16-B activation chunks each thread stages (NX)     */
    int64_t workspace_bytes;  /* split partials, f32 [splits][M][N]                 */
    /* the kernel's limits */
    int32_t xs_elems;         /* staged bf16 activations per block                  */
    int32_t xs_pad_elems;     /* row padding appended to the staging buffer         */
    int32_t kb_max;           /* K range of one block                               */
    int32_t kb_max_e8;        /* K range of one block of the E = 8 instances        */
    int32_t mmax;             /* activation rows                                    */
    int32_t max_waves;
    int32_t sums_rows_e4, sums_cols_e4; /* LDS sub-block sums [rows][cols], E <= 4  */
    int32_t sums_rows_e8, sums_cols_e8; /* the same for E = 8                       */
} thq_gemv_plan_info;

int thq_plan_gemv_mfma(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, thq_gemv_plan_info* out);

/* Prefill / verify GEMM (bf16 rows), for a device with `cus` compute units. */
typedef struct thq_gemm_plan_info {
    int32_t bm;               /* rows per block tile                                */
    int32_t splits;           /* K splits                                           */
    int32_t k_steps;          /* 64-wide K steps per split                          */
    int64_t tiles_n, tiles_m;
    int64_t workspace_bytes;  /* split partials, f32 [splits][M][N]                 */
} thq_gemm_plan_info;

int thq_plan_gemm(int dtype, int exact, int64_t m, int64_t n, int64_t k, int gate_up, int cus,
                  thq_gemm_plan_info* out);

/* Wide exact-weight GEMV (M = 1..64 bf16 rows, K a multiple of 256), for a
 * device with `cus` compute units; the router takes it for 17..64 rows. */
typedef struct thq_wide_plan_info {
    int32_t splits;           /* K splits (0: the shape has no plan)                */
    int32_t chunks_per_split; /* 256-wide K chunks per split                        */
    int64_t workspace_bytes;  /* split partials, f32 [splits][M][N]                 */
} thq_wide_plan_info;

int thq_plan_gemv_wide(int dtype, int64_t m, int64_t n, int64_t k, int cus, thq_wide_plan_info* out);

/* Tile-plane decode GEMV (3..8 bf16 rows of a Q4_K / MLX affine weight
 * with a tile plane, thq_weight_add_tiles), for a device with `cus` compute
 * units; gate_up: the fused [gate; up] weight of thq_gate_up_silu (n rows,
 * n / 2 outputs).  waves 0 for shapes it does not cover (M outside 1..8,
 * K < 256, gate/up halves that are not whole 32-row tiles). */
typedef struct thq_tile_plan_info {
    int32_t waves;            /* waves per block (0: the shape has no plan)        */
    int32_t splits;           /* K splits (partials summed by a reduce launch)      */
    int64_t workspace_bytes;  /* split partials, f32 [splits][M][N]                 */
} thq_tile_plan_info;

int thq_plan_gemv_tile(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, int cus,
                       thq_tile_plan_info* out);

/* Streaming mid-M GEMM with rounded weights (Q4_K / MLX affine on the
 * row-quad plane, bf16 rows, K a multiple of 256), for a device with `cus`
 * compute units; gate_up: the fused [gate; up] weight (n rows, n / 2
 * outputs).  The router takes it for 17..128 rows (17..64 where n < k).
 * group_halves 0 for shapes it does not cover. */
typedef struct thq_mid_plan_info {
    int32_t group_halves;     /* 32-row halves per activation group (2 or 4; 0: no plan) */
    int32_t col_tiles;        /* 32-row column tiles per wave                       */
    int32_t waves;            /* waves per block (4 or 8)                           */
    int32_t groups;           /* activation groups (blocks along M)                 */
    int32_t splits;           /* K splits (partials summed by a reduce launch)      */
    int32_t chunks_per_split; /* 256-wide K chunks per split                        */
    int64_t workspace_bytes;  /* split partials, f32 [splits][M][N]                 */
} thq_mid_plan_info;

int thq_plan_gemm_mid(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, int cus, thq_mid_plan_info* out);

#ifdef __cplusplus
}
#endif
#endif /* THQ_PLAN_H */
