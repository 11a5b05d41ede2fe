// thq_api.cpp — the extern "C" boundary (include/thq.h): device contexts,
// weight lifetime, validation, routing by M, and error reporting.  No C++
// exception crosses the ABI; every entry point returns a THQ_* code.
//
// Routing mirrors the reference's projection router QLin::linear_ps
// (engine/src/qwen35.rs:398-617: m == 1 -> GEMV, m > 1 -> tile kernels,
// inapplicable kernels fall back instead of failing) and candle's
// QMatMul::forward.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/thq.h"
#include "../../include/thq_plan.h"
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

// Device scratch of thq_matmul_noalloc: split-K partials and quantized
// activation planes for callers that cannot allocate.  Each device the
// library runs on holds its own copy until the process ends.  In host code
// this name is a host-side stand-in, not a device address: kernels get the
// address hipGetSymbolAddress returns for the current device (thq_ctx::scratch).
constexpr size_t THQ_NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[THQ_NOALLOC_SCRATCH_BYTES];

struct thq_ctx {
    int device = 0;
    void* scratch = nullptr;  // this device's copy of `scratch` (thq_init)
    int cus = 256;  // compute units (GEMM split planning)
    std::mutex mu;
    void* ws = nullptr;  // workspace: split-K partials, argmax partials, logits
    size_t ws_bytes = 0;
    // buffers the workspace outgrew: kernels already enqueued (or captured in
    // a graph) may still use them, so they live until thq_destroy
    std::vector<void*> retired;
    // arrival counters of the emitting gate/up epilogue: zero between launches
    // (each launch leaves them zero); grown like the workspace
    uint32_t* emit_cnt = nullptr;
    size_t emit_cnt_n = 0;
    // arrival counters of the tile-plane GEMV's last-block split reduction:
    // zero between launches; grown like the workspace
    uint32_t* tile_cnt = nullptr;
    size_t tile_cnt_n = 0;
};

struct thq_weight {
    int device = 0;          // the device that holds q / aux (not the context: a
                             // weight may outlive the context that made it)
    int qtype = 0;           // thq_dtype
    int64_t N = 0, K = 0;
    int gs = 0;              // MLX affine group size
    uint8_t* q = nullptr;    // Q8_0 i8 plane / Q4_K and MLX affine row-quad plane / Q6_K planes
    uint8_t* aux = nullptr;  // Q8_0 f16 scale plane
    uint8_t* tq = nullptr;   // Q4_K / MLX affine tile plane (thq_weight_add_tiles), or null
};

namespace thq {

thread_local std::string g_err;

// the calling thread's last error message (thq_last_error); shared with the
// GGUF reader in thq_gguf.cpp
int fail_v(int code, const char* fmt, va_list ap) {
    char buf[512];
    vsnprintf(buf, sizeof(buf), fmt, ap);
    g_err = buf;
    return code;
}

}  // namespace thq

namespace {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const int rc = thq::fail_v(code, fmt, ap);
    va_end(ap);
    return rc;
}

#define HIP_TRY(expr)                                                                            \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return fail(THQ_EHIP, "%s: %s", #expr, hipGetErrorString(e_));     \
    } while (0)

int block_of(int qtype) {
    switch (qtype) {
        case THQ_Q8_0: return 32;
        case THQ_Q4_K: return 256;
        case THQ_Q6_K: return 256;
        case THQ_MLX_Q4: return 64;
        default: return 0;
    }
}

// GGUF block bytes; for MLX affine weights the QLin arrays (wq + sb)
size_t gguf_bytes(int qtype, int64_t n, int64_t k, int gs = 64) {
    if (qtype == THQ_Q8_0) return (size_t)n * (size_t)(k / 32) * 34;
    if (qtype == THQ_MLX_Q4) return (size_t)n * (size_t)k / 2 + (size_t)n * 2 * (size_t)(k / gs) * 2;
    if (qtype == THQ_Q6_K) return (size_t)n * (size_t)(k / 256) * 210;
    return (size_t)n * (size_t)(k / 256) * 144;
}

// the kernels' type ids: 8 Q8_0, 12 Q4_K, 13 MLX affine on the Q4_K layout, 14 Q6_K
thq::WeightView view(const thq_weight* w) {
    return thq::WeightView{w->qtype == THQ_MLX_Q4 ? 13 : w->qtype, w->N, w->K, w->q, w->aux};
}

// device plane sizes: Q8_0 = i8 tile plane + f16 scale tile plane (rows
// padded to a multiple of 32); Q4_K / MLX affine = one row-quad plane (rows
// padded to a multiple of 4 and, for MLX affine, K to whole superblocks);
// Q6_K = the QL/QH/SC/D planes.  Padding is zero.
size_t q_plane_bytes(int qtype, int64_t n, int64_t k) {
    if (qtype == THQ_Q8_0) return (size_t)thq::q8t_q_bytes(n, k);
    if (qtype == THQ_Q6_K) return thq::q6k_layout(n, k).total;
    return (size_t)((n + 3) / 4) * (size_t)((k + 255) / 256) * 576;
}
size_t aux_plane_bytes(int qtype, int64_t n, int64_t k) {
    return qtype == THQ_Q8_0 ? (size_t)thq::q8t_d_bytes(n, k) : 0;
}

int check_dtype_shape(int dtype, int64_t n, int64_t k) {
    const int bs = block_of(dtype);
    if (!bs)
        return fail(THQ_EDTYPE, "unsupported weight dtype %d (want Q8_0=8, Q4_K=12, Q6_K=14 or MLX_Q4=100)", dtype);
    if (n <= 0 || k <= 0) return fail(THQ_ESHAPE, "weight shape [%lld, %lld] must be positive", (long long)n, (long long)k);
    if (k % bs) return fail(THQ_ESHAPE, "K=%lld is not a multiple of the block size %d", (long long)k, bs);
    if (k > (int64_t)1 << 30 || n > (int64_t)1 << 40) return fail(THQ_ESHAPE, "weight shape too large");
    // the packed bytes (at most 34 B per 32 weights) must stay far from any
    // size or offset wrap: 2^46 B is beyond any device's memory
    if ((double)n * (double)k * (34.0 / 32.0) > (double)((int64_t)1 << 46))
        return fail(THQ_ESHAPE, "weight of %lld x %lld elements is too large", (long long)n, (long long)k);
    return THQ_OK;
}

int alloc_weight(thq_ctx* ctx, int dtype, int64_t n, int64_t k, thq_weight** out) {
    thq_weight* w = new (std::nothrow) thq_weight();
    if (!w) return fail(THQ_ENOMEM, "host allocation failed");
    w->device = ctx->device;
    w->qtype = dtype;
    w->N = n;
    w->K = k;
    const size_t qb = q_plane_bytes(dtype, n, k), ab = aux_plane_bytes(dtype, n, k);
    hipError_t e = hipMalloc((void**)&w->q, qb);
    if (e == hipSuccess && (dtype == THQ_Q4_K || dtype == THQ_MLX_Q4) && (n & 3))
        e = hipMemset(w->q, 0, qb);  // zero padding rows
    if (e == hipSuccess && dtype == THQ_Q8_0 && (n & 31)) e = hipMemset(w->q, 0, qb);
    if (e == hipSuccess && ab) {
        e = hipMalloc((void**)&w->aux, ab);
        // zero padding rows and the padded tail of each row's last 8-block chunk
        if (e == hipSuccess && ((n & 31) || ((k / 32) & 7))) e = hipMemset(w->aux, 0, ab);
        if (e != hipSuccess) (void)hipFree(w->q);
    }
    if (e != hipSuccess) {
        delete w;
        return fail(THQ_ENOMEM, "hipMalloc(%zu + %zu) for weight: %s", qb, ab, hipGetErrorString(e));
    }
    *out = w;
    return THQ_OK;
}

// Grow the context workspace (caller holds ctx->mu).  The old buffer is
// retired, not freed: work already enqueued on any stream, or captured in a
// graph, may still read or write it, so it lives until thq_destroy.  No
// device synchronization is needed.
int ensure_ws(thq_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->ws_bytes) return THQ_OK;
    size_t want = bytes + (bytes >> 3);
    if (want < 2 * ctx->ws_bytes) want = 2 * ctx->ws_bytes;  // retired bytes stay below the live size
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) return fail(THQ_ENOMEM, "workspace hipMalloc(%zu): %s", want, hipGetErrorString(e));
    if (ctx->ws) ctx->retired.push_back(ctx->ws);
    ctx->ws = p;
    ctx->ws_bytes = want;
    return THQ_OK;
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// n zeroed arrival counters of the context (caller holds ctx->mu), grown by
// a synchronous allocation and clear like the workspace; null if that fails
// (the caller then takes the path without counters)
uint32_t* tile_counters(thq_ctx* ctx, int64_t n) {
    if ((size_t)n <= ctx->tile_cnt_n) return ctx->tile_cnt;
    const size_t want = std::max((size_t)n + (size_t)n / 8, 2 * ctx->tile_cnt_n);
    uint32_t* p = nullptr;
    hipError_t e = hipMalloc((void**)&p, want * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(p, 0, want * sizeof(uint32_t));
    if (e != hipSuccess) {
        if (p) (void)hipFree(p);
        return nullptr;
    }
    if (ctx->tile_cnt) ctx->retired.push_back(ctx->tile_cnt);
    ctx->tile_cnt = p;
    ctx->tile_cnt_n = want;
    return p;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// MLX affine weights: K a multiple of 64 and of the group size; groups of
// 64 or any multiple of 64; the tiled QLin form exists for gs = 64 only
int check_affine(int64_t n, int64_t k, int gs, int tiled) {
    int rc = check_dtype_shape(THQ_MLX_Q4, n, k);
    if (rc) return rc;
    if (gs <= 0 || gs % 64 || k % gs)
        return fail(THQ_EDTYPE, "MLX affine group size %d unsupported (a multiple of 64 dividing K=%lld)", gs,
                    (long long)k);
    if (tiled && gs != 64) return fail(THQ_EDTYPE, "the tiled QLin layout has groups of 64");
    return THQ_OK;
}

// bytes of the QLin arrays: row-major or tiled (rows padded to 256)
void affine_src_bytes(int64_t n, int64_t k, int gs, int tiled, size_t& wq_bytes, size_t& sb_bytes) {
    const int64_t rows = tiled ? (n + 255) / 256 * 256 : n;
    wq_bytes = (size_t)rows * (size_t)(k / 8) * 4;
    sb_bytes = (size_t)rows * 2 * (size_t)(k / gs) * 2;
}

hipError_t dequant_any(const thq_weight* w, void* out, bool bf16, hipStream_t s) {
    if (w->qtype == THQ_Q8_0)
        return thq::launch_dequant_q8_0(reinterpret_cast<const int8_t*>(w->q), reinterpret_cast<const uint16_t*>(w->aux),
                                        out, bf16, w->N, w->K / 32, s);
    if (w->qtype == THQ_MLX_Q4) return thq::launch_dequant_affine(w->q, out, bf16, w->N, (int)w->K, s);
    if (w->qtype == THQ_Q6_K) return thq::launch_dequant_q6k(w->q, out, bf16, w->N, (int)(w->K / 256), s);
    return thq::launch_dequant_q4k(w->q, out, bf16, w->N, (int)(w->K / 256), s);
}

// One projection call: the arguments of thq_matmul / thq_gate_up_silu (gu)
// and of the LM head inside thq_matmul_argmax.  With `am` (fused argmax, y
// unused) only a path with the fused epilogue launches; am->nb = 0 reports
// that this shape / type has none and nothing ran.
struct Call {
    thq_ctx* ctx;
    const thq_weight* w;
    const void* x;
    int xt;
    int64_t m;
    void* y;
    int yt;
    uint32_t flags;
    bool gu;
    hipStream_t s;
    thq::AmaxOut* am;
    size_t scratch_cap = SIZE_MAX;  // routes needing more scratch are not planned
    bool counters = true;           // the caller can supply zeroed arrival counters
};

// an environment switch set to "0" (read on every call)
bool env_flag_off(const char* name) {
    const char* e = getenv(name);
    return e && e[0] == '0' && e[1] == 0;
}

// K-split routes sum their partials in the last block of each output tile
// (arrival counters); THQ_TILE_TICKET=0 takes the counter-free path instead
// (partials summed by a separate k_split_reduce launch, bit for bit the same)
bool tickets_on() { return !env_flag_off("THQ_TILE_TICKET"); }

// Arrival counters for the one-launch top-k (32 per row of a launch of at
// most 2048 rows), or null with THQ_TILE_TICKET=0 or when they cannot be
// allocated (the two-launch form then runs; same results).
uint32_t* topk_counters(thq_ctx* ctx, int64_t m, int64_t* n) {
    *n = 0;
    if (!tickets_on()) return nullptr;
    const int64_t want = thq::topk_counters(m);
    uint32_t* p = tile_counters(ctx, want);
    if (p) *n = want;
    return p;
}

int check_call(const Call& c) {
    if (!c.ctx || !c.w) return fail(THQ_EINVAL, "null context or weight");
    if (c.xt != THQ_ACT_F32 && c.xt != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad x_type %d", c.xt);
    if (c.yt != THQ_ACT_F32 && c.yt != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad y_type %d", c.yt);
    if (c.flags & ~(THQ_MODE_EXACT_W | THQ_MODE_Q8ACT)) return fail(THQ_EINVAL, "unknown flags 0x%x", c.flags);
    if (c.m < 0) return fail(THQ_ESHAPE, "M=%lld must be >= 0", (long long)c.m);
    if (c.m > (1 << 24)) return fail(THQ_ESHAPE, "M=%lld too large", (long long)c.m);
    if (c.gu && (c.w->N % 2)) return fail(THQ_ESHAPE, "gate/up weight has an odd row count %lld", (long long)c.w->N);
    if (c.m == 0) return THQ_OK;
    if (!c.x || (!c.y && !c.am)) return fail(THQ_EINVAL, "null x or y");
    if ((c.flags & THQ_MODE_Q8ACT) && !c.am) {
        if (c.w->qtype == THQ_MLX_Q4) return fail(THQ_EDTYPE, "THQ_MODE_Q8ACT applies to GGUF weights only");
        if (c.w->qtype == THQ_Q6_K) return fail(THQ_EDTYPE, "THQ_MODE_Q8ACT is not implemented for Q6_K weights");
        if (!thq::q8act_supported(c.w->qtype, c.w->K))
            return fail(THQ_ESHAPE, "K=%lld too large for THQ_MODE_Q8ACT", (long long)c.w->K);
        if (!aligned16(c.x)) return fail(THQ_EALIGN, "THQ_MODE_Q8ACT needs 16-byte aligned x");
    }
    return THQ_OK;
}

// The kernels a call runs, and the device scratch (split-K partials or the
// quantized activation planes) they use, known before anything launches.
enum class Kind { NONE, Q8ACT, Q8ACT_TILE, GEMV1, ROWS, GEMV_TILE, GEMV_MFMA, GEMV_MFMA_GROUPS, WIDE, GEMM, GEMM_DQ, GEMM_FQ, GEMM_RQ, GEMM_MID, GENERIC };
struct Route {
    Kind kind = Kind::NONE;
    thq::GemvPlan gp;
    thq::GemvPlan gp_last;  // GEMV_MFMA_GROUPS: the plan of the last, partial group of rows
    thq::WidePlan wp;
    thq::TilePlan tp;
    thq::GemmPlan gm;
    thq::FqPlan fq;
    thq::RqPlan rq;
    thq::MidPlan mp;
    bool exact = false;
    size_t scratch = 0;
};

size_t align_up(size_t b, size_t a) { return (b + a - 1) / a * a; }

// THQ_MODE_Q8ACT on a Q4_K weight with a tile plane: 2..8 rows take the
// int8-MFMA tile kernel (THQ_Q8ACT_TILE=0: the row-quad kernel)
thq::TilePlan q8act_tile_plan(const thq_ctx* ctx, const thq_weight* w, int64_t m, bool gu) {
    static const bool on = !env_flag_off("THQ_Q8ACT_TILE");
    if (!on || !w->tq || w->qtype != THQ_Q4_K || m < 2 || m > 8) return thq::TilePlan{};
    return thq::plan_gemv_tile(m, w->N, w->K, gu, ctx->cus);
}

// Routing by rows, as QLin::linear_ps (engine/src/qwen35.rs:398-617).  A
// validated call with m >= 1.  Kind::NONE: a fused-argmax call whose route
// has no fused epilogue (nothing to launch).
Route plan_route(const Call& c) {
    Route r;
    const thq_weight* w = c.w;
    const int64_t m = c.m;
    const thq::WeightView v = view(w);
    const bool xf32 = c.xt == THQ_ACT_F32;
    const int64_t nout = c.gu ? w->N / 2 : w->N;
    if (c.flags & THQ_MODE_Q8ACT) {
        if (c.am) return r;
        r.kind = Kind::Q8ACT;
        r.scratch = thq::q8act_workspace_bytes(w->qtype, m, w->K);
        const thq::TilePlan tp = q8act_tile_plan(c.ctx, w, m, c.gu);
        if (tp.kw > 0) {
            // the Q8_K planes, then the split partials
            r.kind = Kind::Q8ACT_TILE;
            r.tp = tp;
            r.scratch = align_up(r.scratch, 256) + tp.workspace_bytes;
        }
        return r;
    }
    // M = 1 keeps the VALU GEMV unless THQ_GEMV_M1=mfma; 2..16 bf16 rows go to the MFMA GEMV
    static const bool m1_mfma = [] {
        const char* e = getenv("THQ_GEMV_M1");
        return e && !strcmp(e, "mfma");
    }();
    const bool q6 = w->qtype == THQ_Q6_K;
    const thq::GemvPlan gp = (!xf32 && aligned16(c.x) && m <= 16)
                                 ? thq::plan_gemv_mfma(v.qtype, m, w->N, w->K, c.gu)
                                 : thq::GemvPlan{};
    const bool skinny = gp.waves > 0;
    // the 4-bit tile kernels need whole superblocks (MLX affine K % 256 != 0 runs the generic kernel)
    const bool q4 = w->qtype == THQ_Q4_K || w->qtype == THQ_MLX_Q4;
    // 2..4 bf16 rows of Q4_K / MLX affine at K <= 4096: the VALU row kernel (THQ_GEMV_ROWS=0: MFMA)
    static const bool rows_on = [] {
        const char* e = getenv("THQ_GEMV_ROWS");
        return !(e && !strcmp(e, "0"));
    }();
    // 17..64 bf16 rows (fewer on the widest outputs, below): the wide exact-weight GEMV where exact weights are
    // required (Q8_0 up to 64 rows, THQ_MODE_EXACT_W on 4- / 6-bit weights)
    // and on outputs wide enough to fill the GPU without splitting K (the
    // verify LM head); THQ_GEMV_WIDE=0 turns it off
    static const bool wide_on = [] {
        const char* e = getenv("THQ_GEMV_WIDE");
        return !(e && !strcmp(e, "0"));
    }();
    // On outputs that fill the GPU without splitting K (the verify LM head,
    // 151936 x 4096) it also takes fewer rows, ahead of the MFMA decode GEMV:
    // from 4 rows of Q8_0, 5 of Q4_K / affine, 9 of Q6_K (151936 x 4096 at
    // M = 3..16: Q8_0 128-136 against 129-157 us, Q4_K 99-104 against 95-147,
    // Q6_K 163-167 against 147-198).  THQ_WIDE_MIN_M sets the lowest row count.
    static const int wide_env = [] {
        const char* e = getenv("THQ_WIDE_MIN_M");
        return e && *e ? atoi(e) : 0;
    }();
    int wide_min_m = 17;
    if (nout >= 65536) wide_min_m = w->qtype == THQ_Q8_0 ? 4 : (w->qtype == THQ_Q6_K ? 9 : 5);
    if (wide_env > 0) wide_min_m = wide_env < 2 ? 2 : wide_env;
    const thq::WidePlan wp = (wide_on && !xf32 && aligned16(c.x) && m >= wide_min_m && m <= 64)
                                 ? thq::plan_gemv_wide(v.qtype, m, w->N, w->K, c.ctx->cus)
                                 : thq::WidePlan{};
    // 17..32 rows of Q4_K / MLX affine / Q6_K: the wide GEMV (exact
    // weights) is also the fastest route (12288 x 4096 / 4096 x 12288 /
    // gate/up 2 x 12288 x 4096 at M = 17..32: Q4_K 19.2-20.5 / 21.0-21.5 /
    // 30.2-31.1 us against the streaming GEMM's 24.5-25.0 / 26.3-26.6 /
    // 36.1-43.8; Q6_K 27.0-27.7 / 27.0-27.4 against the tile GEMM's 30.0-30.1
    // / 32.4-33.2; from 40-48 rows it is slower); THQ_GEMM_MID=1 keeps the
    // 4-bit formats' rows on the streaming GEMM
    const char* mde0 = getenv("THQ_GEMM_MID");
    const bool mid_forced = mde0 && !strcmp(mde0, "1");
    const bool wide_ok = wp.splits > 0 && (w->qtype == THQ_Q8_0 || (c.flags & THQ_MODE_EXACT_W) || nout >= 65536 ||
                                           (((q4 && !mid_forced) || q6) && m <= 32));
    // Q8_0 at M = 1 from 12288 outputs: the MFMA GEMV on the tile layout beats
    // the VALU kernel (bf16 x; 12288 / 24576 x 4096: 13.7 / 21.9 vs 14.0 /
    // 23.1 us; LM head 151936 x 4096: 111 vs 125 us); below, the VALU kernel
    // (3072 x 1024 / 4096 x 4096 / 6144 x 4096: 3.2 / 7.7 / 8.4 vs 5.7 / 8.2 / 9.7 us)
    const bool q8_m1_mfma = w->qtype == THQ_Q8_0 && nout >= 12288;
    // a weight with a tile plane: 3..8 bf16 rows take the tile-plane GEMV
    // (whole-line loads; gate/up when each half is a whole number of tiles;
    // THQ_TILE_MIN_M moves the lower bound, 2 makes M = 2 take it instead of
    // the row kernel)
    static const int tile_min_m = [] {
        const char* e = getenv("THQ_TILE_MIN_M");
        const int v = e && *e ? atoi(e) : 3;
        return v < 1 ? 1 : v;
    }();
    const thq::TilePlan tp = (w->tq && q4 && !c.am && !xf32 && aligned16(c.x) && m >= tile_min_m && m <= 8)
                                 ? thq::plan_gemv_tile(m, w->N, w->K, c.gu, c.ctx->cus)
                                 : thq::TilePlan{};
    if (tp.kw > 0) {
        r.kind = Kind::GEMV_TILE;
        r.tp = tp;
        r.scratch = tp.workspace_bytes;
        return r;
    }
    if (m == 1 && !((m1_mfma || q8_m1_mfma) && skinny) && aligned16(c.x) &&
        thq::gemv1_supported(v.qtype, (int)w->K, c.gu, w->N)) {
        r.kind = Kind::GEMV1;
    } else if (rows_on && !xf32 && aligned16(c.x) && thq::gemv_rows_supported(v.qtype, (int)m, (int)w->K, c.gu, w->N) &&
               // 3..4 rows over >= 12288 outputs: the MFMA GEMV is faster (12288 x 4096,
               // M = 3 / 4: 13.04 / 13.20 against 13.41 / 13.63 us; gate/up 2 x 12288:
               // 19.45 against 20.45 us); at 4096 outputs the row kernel is (6.8 against 8.2 us)
               !(m >= 3 && skinny && nout >= 12288)) {
        if (!c.am) r.kind = Kind::ROWS;
    } else if (skinny && !(wide_ok && m >= wide_min_m)) {
        // the fused epilogue exists on the unsplit plan only (no scratch)
        if (!c.am || gp.splits == 1) {
            r.kind = Kind::GEMV_MFMA;
            r.gp = gp;
            r.scratch = c.am ? 0 : gp.workspace_bytes;
        }
    } else if (wide_ok) {
        if (!c.am || wp.splits == 1) {
            r.kind = Kind::WIDE;
            r.wp = wp;
            r.scratch = c.am ? 0 : wp.workspace_bytes;
        }
    } else if (c.am) {
        // no fused epilogue
    } else if (!xf32 && aligned16(c.x) && w->K % 64 == 0 &&  // the GEMMs step K in 64-wide tiles
               // gate/up rows of < 256 outputs: the rounded-weight tile's error, seen
               // through silu(g)*u, is not averaged down by the row norm (the exact
               // kernel costs nothing at that size)
               !(c.gu && nout < 256) &&
               // exact Q6_K has no GEMM tile (its exact path is the decode GEMV in
               // groups of 16 rows); exact Q4_K / MLX affine run k_gemm's exact
               // tile (THQ_EXACT_GEMM=0: the groups of 16 rows instead)
               !((q4 || q6) && w->K % 256) &&
               !((q6 || (q4 && env_flag_off("THQ_EXACT_GEMM"))) && (c.flags & THQ_MODE_EXACT_W)) &&
               !(q6 && (m <= 8 || thq::q6k_layout(w->N, w->K).total >= (1ull << 32) ||
                        (uint64_t)m * (uint64_t)w->K * 2 >= (1ull << 32)))) {
        r.kind = Kind::GEMM;
        r.exact = (c.flags & THQ_MODE_EXACT_W) || (w->qtype == THQ_Q8_0 && m <= 64);
        r.gm = thq::plan_gemm(v.qtype, r.exact, m, w->N, w->K, c.gu, c.ctx->cus);
        r.scratch = r.gm.workspace_bytes;
        // many rows of a plain projection: dequantize the weight to bf16 once
        // and run the bf16 GEMM (the reference's "dequant + bf16 matmul"
        // prefill route): the tile kernel repeats its dequantization per
        // 256-row block, and on gfx950 that VALU work adds to the MFMA time
        // (12288 x 4096 at M = 2048: Q4_K 203 against 258 us, Q6_K 214 / 274,
        // MLX affine 207 / 236, Q8_0 215 / 241).  Only from 1024 rows and
        // where its 256 x 384 tiles fill the GPU, since it has no split-K:
        // all CUs, or two thirds of them for Q4_K / Q6_K, whose in-tile
        // dequantization costs the most (4096 x 12288 at M = 4096, 176 tiles:
        // Q4_K 429 against 449 us, Q6_K 436 / 501, Q8_0 452 / 439, affine
        // 434 / 429; 12288 x 4096 at M = 1024, 128 tiles: Q4_K 168 / 153).
        // THQ_GEMM_DQ: 0 never, 1 wherever supported (tests), unset: that rule
        const char* dqe = getenv("THQ_GEMM_DQ");
        const int dq_mode = dqe && *dqe ? atoi(dqe) : -1;
        const size_t wb_bytes = round256((size_t)w->N * (size_t)w->K * 2);
        // the bf16 weight lives in the context workspace, which keeps its size
        // until thq_destroy: weights above THQ_DQ_MAX_MB (default 512 MiB of
        // bf16, e.g. a 151936 x 4096 LM head at 1.2 GiB) stay on the tile GEMM
        const char* dqm = getenv("THQ_DQ_MAX_MB");
        const size_t dq_cap = (size_t)(dqm && *dqm ? atoll(dqm) : 512) << 20;
        const int64_t blocks = thq::gemm_b16_blocks(m, w->N), cus = c.ctx->cus;
        const bool q4k_or_q6k = w->qtype == THQ_Q4_K || w->qtype == THQ_Q6_K;
        if (!r.exact && !c.gu && dq_mode != 0 && thq::gemm_b16_supported(m, w->N, w->K) &&
            wb_bytes <= c.scratch_cap && wb_bytes <= dq_cap &&
            (dq_mode == 1 || (m >= 1024 && (q4k_or_q6k ? 3 * blocks >= 2 * cus : blocks >= cus)))) {
            r.kind = Kind::GEMM_DQ;
            r.scratch = wb_bytes;
        }
        // Q4_K / MLX affine with rounded weights: the GEMM that dequantizes
        // its weight tiles into LDS (k_gemm_fq).  THQ_GEMM_FQ: 0 never,
        // 1 wherever supported, unset: off
        const char* fqe = getenv("THQ_GEMM_FQ");
        const int fq_mode = fqe && *fqe ? atoi(fqe) : 0;
        if (q4 && !r.exact && fq_mode == 1 && thq::gemm_fq_supported(m, w->N, w->K, c.gu)) {
            const thq::FqPlan fp = thq::plan_gemm_fq(m, w->N, w->K, c.gu, c.ctx->cus);
            if (fp.workspace_bytes <= c.scratch_cap) {
                r.kind = Kind::GEMM_FQ;
                r.fq = fp;
                r.scratch = fp.workspace_bytes;
            }
        }
        // Q4_K / MLX affine with rounded weights from 1024 rows: the GEMM that
        // dequantizes each wave's 32 weight rows in registers (k_gemm_rq), in
        // place of the tile GEMM (12288 x 4096 at M = 1024: 116 against 144 us;
        // 4096 x 12288 at M = 2048: 209 against 219 us) and, for weights with
        // fewer rows than columns (the down projection), of the dequantize-
        // then-GEMM route (4096 x 12288 at M = 4096: 369 against 388 us;
        // 12288 x 4096 keeps that route: 180 against 219 us at M = 2048); on
        // weights of at least 12288 x 4096 elements also from 768 rows, and
        // gate/up from 384 (12288 x 4096 / 4096 x 12288 at M = 768: 107.6 /
        // 106.7 against 136.3 / 115.4 us; gate/up 2 x 12288 x 4096 at M = 384
        // / 512: 128.4 / 130.4 against 146.5 / 151.3 us; at M = 512 the plain
        // shapes keep the tile GEMM: 72.0 / 70.9 against 78.8 / 84.9).  Its
        // K splits meet in the last block of each tile, so only with arrival
        // counters.  THQ_GEMM_RQ: 0 never, 1 wherever supported (tests),
        // unset: that rule
        const char* rqe = getenv("THQ_GEMM_RQ");
        const int rq_mode = rqe && *rqe ? atoi(rqe) : -1;
        const bool rq_big = w->N * w->K >= (int64_t)12288 * 4096 && r.kind == Kind::GEMM &&
                            (m >= 768 || (c.gu && m >= 384));
        const bool rq_default = rq_big || (m >= 1024 && (r.kind == Kind::GEMM ||
                                                         (r.kind == Kind::GEMM_DQ && dq_mode == -1 && w->N < w->K)));
        if (q4 && !r.exact && r.kind != Kind::GEMM_FQ && rq_mode != 0 && (rq_mode == 1 || rq_default) &&
            c.counters && tickets_on() &&
            thq::gemm_rq_supported(w->qtype == THQ_MLX_Q4 ? 13 : 12, m, w->N, w->K, c.gu)) {
            const thq::RqPlan rp = thq::plan_gemm_rq(m, w->N, w->K, c.gu, c.ctx->cus);
            // the counters thq_reserve documents (one per 32 rows of the weight) cover its tiles
            if (rp.workspace_bytes <= c.scratch_cap && rp.counters <= (w->N + 31) / 32) {
                r.kind = Kind::GEMM_RQ;
                r.rq = rp;
                r.scratch = rp.workspace_bytes;
            }
        }
        // Q4_K / MLX affine with rounded weights at tens of rows (past the
        // 32 the wide GEMV takes): the streaming GEMM (k_gemm_mid: each wave's
        // weight rows straight into registers, the activation rows copied
        // into LDS), up to 128 rows on weights with at least as many rows as
        // columns and up to 64 on the others (12288 x 4096 at M = 48 / 64 /
        // 96 / 128: 25.2 / 25.9 / 33.6 / 34.7 against 28.1 / 28.9 / 42.0 /
        // 37.2 us; gate/up 2 x 12288 x 4096 at M = 64 / 128: 38.8 / 51.1
        // against 46.2 / 56.9 us; 4096 x 12288 at M = 64: 26.3 against 28.8 us,
        // at M = 128: 35.2 against 33.0 us), and up to 384 rows on square
        // weights of at most 4096 rows, where the tile GEMM's few tiles leave
        // CUs idle (4096 x 4096 at M = 160 / 256 / 384: 23.6 / 26.1 / 31.9
        // against 27.5 / 31.0 / 34.6 us; at 512: 36.9 against 35.6).
        // THQ_GEMM_MID: 0 never, 1 wherever supported (tests), unset: that rule
        const char* mde = getenv("THQ_GEMM_MID");
        const int mid_mode = mde && *mde ? atoi(mde) : -1;
        const int mid_max = w->N >= w->K ? (w->N == w->K && w->N <= 4096 ? 384 : 128) : 64;
        const bool mid_default = m >= 17 && m <= mid_max && r.kind == Kind::GEMM;
        if (q4 && !r.exact && mid_mode != 0 && (mid_mode == 1 || mid_default)) {
            const thq::MidPlan mp = thq::plan_gemm_mid(v.qtype, m, w->N, w->K, c.gu, c.ctx->cus);
            if (mp.mh > 0 && mp.workspace_bytes <= c.scratch_cap) {
                r.kind = Kind::GEMM_MID;
                r.mp = mp;
                r.scratch = mp.workspace_bytes;
            }
        }
    } else if (!xf32 && aligned16(c.x) && (q4 || q6) && m > 16 && w->K % 256 == 0 &&
               thq::plan_gemv_mfma(v.qtype, 16, w->N, w->K, c.gu).waves > 0) {
        // exact 4- / 6-bit weights past the decode GEMV's 16 rows (the verify
        // LM head of batched drafts; the GEMMs round these weights to bf16):
        // the exact decode GEMV over groups of 16 rows, each group streaming
        // the weights again (Q6_K 151936 x 4096, M = 40: 3 groups against
        // the generic kernel's 3.4 ms)
        r.kind = Kind::GEMV_MFMA_GROUPS;
        r.gp = thq::plan_gemv_mfma(v.qtype, 16, w->N, w->K, c.gu);
        r.gp_last = (m % 16) ? thq::plan_gemv_mfma(v.qtype, m % 16, w->N, w->K, c.gu) : r.gp;
        r.scratch = std::max(r.gp.workspace_bytes, r.gp_last.workspace_bytes);
        if (!r.gp_last.waves) r.kind = Kind::GENERIC;
    } else {
        r.kind = Kind::GENERIC;
    }
    return r;
}

// Launch a planned route; `scratch` holds at least r.scratch bytes; `cnt`:
// zeroed arrival counters for the routes that reduce K splits in their last
// block (null: those routes launch a separate reduce).
int exec_route(const Call& c, const Route& r, void* scratch, uint32_t* cnt = nullptr) {
    const thq_weight* w = c.w;
    const thq::WeightView v = view(w);
    const bool xf32 = c.xt == THQ_ACT_F32, yf32 = c.yt == THQ_ACT_F32;
    const int64_t nout = c.gu ? w->N / 2 : w->N;
    const int64_t up_off = c.gu ? w->N / 2 : 0;
    const int m = (int)c.m;
    hipError_t e = hipSuccess;
    switch (r.kind) {
        case Kind::NONE: return THQ_OK;
        case Kind::Q8ACT:
            e = thq::launch_q8act(v, c.x, xf32, c.y, yf32, c.gu, m, nout, up_off, scratch, c.s);
            break;
        case Kind::Q8ACT_TILE: {
            char* planes = static_cast<char*>(scratch);
            float* part = reinterpret_cast<float*>(planes + align_up(thq::q8act_workspace_bytes(w->qtype, m, w->K), 256));
            e = thq::launch_q8act_tiled(r.tp, v, w->tq, c.x, xf32, c.y, yf32, c.gu, m, planes, part, cnt, c.s);
            break;
        }
        case Kind::GEMV1: e = thq::launch_gemv1(v, c.x, xf32, c.y, yf32, c.gu, nout, up_off, c.s, c.am); break;
        case Kind::ROWS: e = thq::launch_gemv_rows(v, c.x, c.y, yf32, c.gu, m, nout, up_off, c.s); break;
        case Kind::GEMV_TILE:
            e = thq::launch_gemv_tile(r.tp, v, w->tq, c.x, c.y, yf32, c.gu, m, static_cast<float*>(scratch), cnt,
                                      c.s);
            break;
        case Kind::GEMV_MFMA:
            e = thq::launch_gemv_mfma(r.gp, v, c.x, c.y, yf32, c.gu, m, nout, up_off, static_cast<float*>(scratch),
                                      c.s, c.am);
            break;
        case Kind::GEMV_MFMA_GROUPS: {
            // groups run in stream order, so they share the scratch
            const size_t xrow = (size_t)w->K * (xf32 ? 4 : 2), yrow = (size_t)nout * (yf32 ? 4 : 2);
            for (int r0 = 0; r0 < m && e == hipSuccess; r0 += 16) {
                const int mm = m - r0 < 16 ? m - r0 : 16;
                e = thq::launch_gemv_mfma(mm == 16 ? r.gp : r.gp_last, v, static_cast<const char*>(c.x) + r0 * xrow,
                                          static_cast<char*>(c.y) + r0 * yrow, yf32, c.gu, mm, nout, up_off,
                                          static_cast<float*>(scratch), c.s, nullptr);
            }
            break;
        }
        case Kind::WIDE:
            e = thq::launch_gemv_wide(r.wp, v, c.x, c.y, yf32, c.gu, m, nout, up_off, static_cast<float*>(scratch),
                                      c.s, c.am);
            break;
        case Kind::GEMM:
            e = thq::launch_gemm(r.gm, v, c.x, c.y, yf32, c.gu, r.exact, m, static_cast<float*>(scratch), c.s);
            break;
        case Kind::GEMM_FQ:
            e = thq::launch_gemm_fq(r.fq, w->qtype == THQ_MLX_Q4, w->q, c.x, c.y, yf32, c.gu, m, w->N, (int)w->K,
                                    static_cast<float*>(scratch), c.s);
            break;
        case Kind::GEMM_RQ:
            e = thq::launch_gemm_rq(r.rq, w->qtype == THQ_MLX_Q4, w->q, c.x, c.y, yf32, c.gu, m, w->N, (int)w->K,
                                    static_cast<float*>(scratch), cnt, c.s);
            break;
        case Kind::GEMM_MID:
            e = thq::launch_gemm_mid(r.mp, v, c.x, c.y, yf32, c.gu, m, nout, up_off, static_cast<float*>(scratch), c.s);
            break;
        case Kind::GEMM_DQ:
            // the weight as bf16 [N][K] in the scratch, then x . Wb^T
            e = dequant_any(w, scratch, true, c.s);
            if (e == hipSuccess) e = thq::launch_gemm_b16(c.x, scratch, c.y, yf32, m, (int)w->N, (int)w->K, c.s);
            break;
        case Kind::GENERIC: e = thq::launch_generic(v, c.x, xf32, c.y, yf32, c.gu, m, nout, up_off, c.s); break;
    }
    if (e != hipSuccess) return fail(THQ_EHIP, "kernel launch: %s", hipGetErrorString(e));
    return THQ_OK;
}

// Validate, plan and launch one call with the context workspace as scratch.
int run_matmul(const Call& c) {
    int rc = check_call(c);
    if (rc || c.m == 0) return rc;
    if (c.am) c.am->nb = 0;
    DeviceGuard g(c.ctx->device);
    const Route r = plan_route(c);
    if (r.kind == Kind::NONE) return THQ_OK;
    std::lock_guard<std::mutex> lk(c.ctx->mu);
    if (r.scratch) {
        rc = ensure_ws(c.ctx, r.scratch);
        if (rc) return rc;
    }
    uint32_t* cnt = nullptr;
    if ((r.kind == Kind::GEMV_TILE || r.kind == Kind::Q8ACT_TILE) && r.tp.splits > 1 && tickets_on())
        cnt = tile_counters(c.ctx, (c.w->N + 31) / 32);  // >= output tiles
    if (r.kind == Kind::GEMM_RQ && r.rq.splits > 1) {
        cnt = tile_counters(c.ctx, (c.w->N + 31) / 32);  // >= r.rq.counters (planned so)
        if (!cnt) return fail(THQ_ENOMEM, "arrival counters: allocation failed");
    }
    return exec_route(c, r, c.ctx->ws, cnt);
}

}  // namespace

extern "C" {

const char* thq_last_error(void) { return thq::g_err.c_str(); }

const char* thq_version(void) { return "thq 0.1 gfx950"; }

int thq_init(int device, thq_ctx** out) {
    if (!out) return fail(THQ_EINVAL, "null out");
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(THQ_EINVAL, "device %d out of range (%d devices)", device, count);
    thq_ctx* c = new (std::nothrow) thq_ctx();
    if (!c) return fail(THQ_ENOMEM, "host allocation failed");
    c->device = device;
    {
        DeviceGuard g(device);
        hipError_t e = hipGetSymbolAddress(&c->scratch, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            delete c;
            return fail(THQ_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        }
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        c->cus = cus;
    *out = c;
    return THQ_OK;
}

void thq_destroy(thq_ctx* ctx) {
    if (!ctx) return;
    if (ctx->ws || ctx->emit_cnt || ctx->tile_cnt || !ctx->retired.empty()) {
        DeviceGuard g(ctx->device);
        (void)hipDeviceSynchronize();
        if (ctx->ws) (void)hipFree(ctx->ws);
        if (ctx->emit_cnt) (void)hipFree(ctx->emit_cnt);
        if (ctx->tile_cnt) (void)hipFree(ctx->tile_cnt);
        for (void* p : ctx->retired) (void)hipFree(p);
    }
    delete ctx;
}

int thq_weight_upload(thq_ctx* ctx, thq_dtype dtype, const void* host_blocks, int64_t n, int64_t k,
                      thq_weight** out) {
    if (!ctx || !host_blocks || !out) return fail(THQ_EINVAL, "null argument");
    if (dtype == THQ_MLX_Q4) return fail(THQ_EDTYPE, "MLX affine weights load with thq_affine_upload");
    int rc = check_dtype_shape(dtype, n, k);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const size_t bytes = gguf_bytes(dtype, n, k);
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, bytes);
    if (e != hipSuccess) return fail(THQ_ENOMEM, "hipMalloc staging(%zu): %s", bytes, hipGetErrorString(e));
    e = hipMemcpy(staging, host_blocks, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(staging);
        return fail(THQ_EHIP, "hipMemcpy weight: %s", hipGetErrorString(e));
    }
    rc = thq_weight_from_device(ctx, dtype, staging, n, k, nullptr, out);  // synchronizes
    (void)hipFree(staging);
    return rc;
}

int thq_weight_from_device(thq_ctx* ctx, thq_dtype dtype, const void* dev_blocks, int64_t n, int64_t k, void* stream,
                           thq_weight** out) {
    if (!ctx || !dev_blocks || !out) return fail(THQ_EINVAL, "null argument");
    if (dtype == THQ_MLX_Q4) return fail(THQ_EDTYPE, "MLX affine weights load with thq_affine_from_device");
    int rc = check_dtype_shape(dtype, n, k);
    if (rc) return rc;
    // the repack kernels read Q4_K blocks as 16-B vectors, Q8_0 / Q6_K blocks as 2-B words
    const uintptr_t need = dtype == THQ_Q4_K ? 16 : 2;
    if ((uintptr_t)dev_blocks % need)
        return fail(THQ_EALIGN, "dev_blocks must be %d-byte aligned for this dtype", (int)need);
    DeviceGuard g(ctx->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    thq_weight* w = nullptr;
    rc = alloc_weight(ctx, dtype, n, k, &w);
    if (rc) return rc;
    const uint8_t* src = static_cast<const uint8_t*>(dev_blocks);
    hipError_t e;
    if (dtype == THQ_Q4_K)
        e = thq::launch_repack_q4k(src, w->q, n, (int)(k / 256), s);
    else if (dtype == THQ_Q6_K)
        e = thq::launch_repack_q6k(src, w->q, n, (int)(k / 256), s);
    else
        e = thq::launch_repack_q8_0(src, reinterpret_cast<int8_t*>(w->q), reinterpret_cast<uint16_t*>(w->aux), n,
                                    k / 32, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        thq_weight_free(w);
        return fail(THQ_EHIP, "weight repack: %s", hipGetErrorString(e));
    }
    *out = w;
    return THQ_OK;
}

int thq_quantize(thq_ctx* ctx, thq_dtype dtype, const float* w_dev, int64_t n, int64_t k, void* stream,
                 thq_weight** out) {
    if (!ctx || !w_dev || !out) return fail(THQ_EINVAL, "null argument");
    if (dtype == THQ_MLX_Q4) return fail(THQ_EDTYPE, "no MLX affine quantizer (the engine loads MLX checkpoints)");
    if (dtype == THQ_Q6_K) return fail(THQ_EDTYPE, "no Q6_K quantizer (Q6_K tensors are read from GGUF files)");
    int rc = check_dtype_shape(dtype, n, k);
    if (rc) return rc;
    if (!aligned16(w_dev)) return fail(THQ_EALIGN, "w_dev must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    thq_weight* w = nullptr;
    rc = alloc_weight(ctx, dtype, n, k, &w);
    if (rc) return rc;
    hipError_t e = dtype == THQ_Q8_0
                       ? thq::launch_quantize_q8_0(w_dev, reinterpret_cast<int8_t*>(w->q),
                                                   reinterpret_cast<uint16_t*>(w->aux), n, k / 32, s)
                       : thq::launch_quantize_q4k(w_dev, w->q, n, (int)(k / 256), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        thq_weight_free(w);
        return fail(THQ_EHIP, "quantize: %s", hipGetErrorString(e));
    }
    *out = w;
    return THQ_OK;
}

int thq_weight_fuse(thq_ctx* ctx, const thq_weight* const* parts, int nparts, thq_weight** out) {
    if (!ctx || !parts || nparts <= 0 || !out) return fail(THQ_EINVAL, "null argument or no parts");
    int64_t n = 0;
    for (int i = 0; i < nparts; ++i) {
        if (!parts[i]) return fail(THQ_EINVAL, "part %d is null", i);
        if (parts[i]->qtype != parts[0]->qtype) return fail(THQ_EDTYPE, "part %d dtype differs", i);
        if (parts[i]->gs != parts[0]->gs) return fail(THQ_EDTYPE, "part %d group size differs", i);
        if (parts[i]->K != parts[0]->K)
            return fail(THQ_ESHAPE, "part %d has K=%lld, part 0 has K=%lld", i, (long long)parts[i]->K,
                        (long long)parts[0]->K);
        n += parts[i]->N;
    }
    const int dtype = parts[0]->qtype;
    const int64_t k = parts[0]->K;
    DeviceGuard g(ctx->device);
    thq_weight* w = nullptr;
    int rc = alloc_weight(ctx, dtype, n, k, &w);
    if (rc) return rc;
    w->gs = parts[0]->gs;
    int64_t row0 = 0;
    for (int i = 0; i < nparts; ++i) {
        hipError_t e = hipSuccess;
        if (dtype == THQ_Q6_K) {
            // each plane is row-major: copy the part's rows of all four
            const thq::Q6Layout dl = thq::q6k_layout(n, k), sl = thq::q6k_layout(parts[i]->N, k);
            const size_t doff[4] = {0, dl.qh, dl.sc, dl.d}, soff[4] = {0, sl.qh, sl.sc, sl.d};
            const size_t rowb[4] = {(size_t)k / 2, (size_t)k / 4, (size_t)k / 16, (size_t)(k / 256) * 2};
            for (int pl = 0; pl < 4 && e == hipSuccess; ++pl)
                e = hipMemcpy(w->q + doff[pl] + (size_t)row0 * rowb[pl], parts[i]->q + soff[pl],
                              (size_t)parts[i]->N * rowb[pl], hipMemcpyDeviceToDevice);
        } else if (dtype != THQ_Q8_0) {
            e = thq::launch_q4k_copy_rows(parts[i]->q, parts[i]->N, w->q, row0, (int)((k + 255) / 256), nullptr);
        } else {
            // tile planes: row by row (a part need not end on a tile boundary)
            e = thq::launch_q8_0_copy_rows(reinterpret_cast<const int8_t*>(parts[i]->q),
                                           reinterpret_cast<const uint16_t*>(parts[i]->aux), parts[i]->N,
                                           reinterpret_cast<int8_t*>(w->q), reinterpret_cast<uint16_t*>(w->aux), row0,
                                           k / 32, nullptr);
        }
        row0 += parts[i]->N;
        if (e != hipSuccess) {
            thq_weight_free(w);
            return fail(THQ_EHIP, "fuse copy: %s", hipGetErrorString(e));
        }
    }
    hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        thq_weight_free(w);
        return fail(THQ_EHIP, "fuse: %s", hipGetErrorString(e));
    }
    *out = w;
    return THQ_OK;
}

int thq_weight_add_tiles(thq_ctx* ctx, thq_weight* w) {
    if (!ctx || !w) return fail(THQ_EINVAL, "null argument");
    if (w->qtype != THQ_Q4_K && w->qtype != THQ_MLX_Q4)
        return fail(THQ_EDTYPE, "tile planes exist for Q4_K and MLX affine weights (dtype %d)", w->qtype);
    if (w->device != ctx->device)
        return fail(THQ_EINVAL, "weight on device %d, context on device %d", w->device, ctx->device);
    if (w->tq) return THQ_OK;
    DeviceGuard g(ctx->device);
    const size_t bytes = thq::tile_plane_bytes(w->N, w->K);
    uint8_t* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(THQ_ENOMEM, "tile plane hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    e = thq::launch_repack_q4t(w->q, p, w->N, w->K, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return fail(THQ_EHIP, "tile plane repack: %s", hipGetErrorString(e));
    }
    w->tq = p;
    return THQ_OK;
}

void thq_weight_free(thq_weight* w) {
    if (!w) return;
    DeviceGuard g(w->device);
    if (w->q) (void)hipFree(w->q);
    if (w->aux) (void)hipFree(w->aux);
    if (w->tq) (void)hipFree(w->tq);
    delete w;
}

int thq_weight_info(const thq_weight* w, thq_dtype* dtype, int64_t* n, int64_t* k, size_t* bytes) {
    if (!w) return fail(THQ_EINVAL, "null weight");
    if (dtype) *dtype = (thq_dtype)w->qtype;
    if (n) *n = w->N;
    if (k) *k = w->K;
    if (bytes) *bytes = gguf_bytes(w->qtype, w->N, w->K, w->gs);
    return THQ_OK;
}

int thq_weight_download(const thq_weight* w, void* host_blocks) {
    if (!w || !host_blocks) return fail(THQ_EINVAL, "null argument");
    if (w->qtype == THQ_MLX_Q4) return fail(THQ_EDTYPE, "MLX affine weights download with thq_affine_download");
    DeviceGuard g(w->device);
    std::vector<uint8_t> qs(q_plane_bytes(w->qtype, w->N, w->K));
    std::vector<uint8_t> aux(aux_plane_bytes(w->qtype, w->N, w->K));
    HIP_TRY(hipMemcpy(qs.data(), w->q, qs.size(), hipMemcpyDeviceToHost));
    if (!aux.empty()) HIP_TRY(hipMemcpy(aux.data(), w->aux, aux.size(), hipMemcpyDeviceToHost));
    uint8_t* dst = static_cast<uint8_t*>(host_blocks);
    if (w->qtype == THQ_Q6_K) {
        const int64_t nsb = w->K / 256;
        const thq::Q6Layout L = thq::q6k_layout(w->N, w->K);
        for (int64_t n = 0; n < w->N; ++n) {
            for (int64_t s = 0; s < nsb; ++s) {
                uint8_t* blk = dst + (n * nsb + s) * 210;
                // undo the regrouping by 64-weight step (thq_dev.hpp, q6k_layout)
                const uint8_t* QL = qs.data() + n * (w->K / 2) + s * 128;
                const uint8_t* QH = qs.data() + L.qh + n * (w->K / 4) + s * 64;
                for (int h = 0; h < 2; ++h) {
                    const uint8_t* a = QL + 64 * h;  // step 2h
                    const uint8_t* b = a + 32;       // step 2h + 1
                    for (int t = 0; t < 32; ++t) {
                        blk[64 * h + t] = (uint8_t)((a[t] & 0x0F) | ((b[t] & 0x0F) << 4));
                        blk[64 * h + 32 + t] = (uint8_t)((a[t] >> 4) | (b[t] & 0xF0));
                    }
                    // qh[32h + l] bits 2Q: quarter Q = 2e + o is step 2h + e, weight 32o + l
                    for (int l = 0; l < 32; ++l) {
                        uint8_t v = 0;
                        for (int q = 0; q < 4; ++q) {
                            const int w = 32 * (q & 1) + l;
                            v |= (uint8_t)(((QH[16 * (2 * h + (q >> 1)) + (w & 15)] >> (2 * (w >> 4))) & 3) << (2 * q));
                        }
                        blk[128 + 32 * h + l] = v;
                    }
                }
                std::memcpy(blk + 192, qs.data() + L.sc + n * (w->K / 16) + s * 16, 16);
                std::memcpy(blk + 208, qs.data() + L.d + (n * nsb + s) * 2, 2);
            }
        }
        return THQ_OK;
    }
    if (w->qtype == THQ_Q4_K) {
        const int nsb = (int)(w->K / 256);
        for (int64_t n = 0; n < w->N; ++n) {
            for (int s = 0; s < nsb; ++s) {
                uint8_t* blk = dst + (n * nsb + s) * 144;
                uint32_t hw[4];
                for (int p = 0; p < 4; ++p) std::memcpy(&hw[p], qs.data() + thq::q4k_hdword(n, nsb, s, p), 4);
                const uint4 h = thq::q4k_hdr_to_gguf(make_uint4(hw[0], hw[1], hw[2], hw[3]));
                std::memcpy(blk, &h, 16);
                for (int c = 0; c < 8; ++c)
                    std::memcpy(blk + 16 + 16 * c, qs.data() + thq::q4k_piece(n, nsb, s, c & 1, c >> 1), 16);
            }
        }
        return THQ_OK;
    }
    const int64_t nb = w->K / 32;
    for (int64_t n = 0; n < w->N; ++n)
        for (int64_t j = 0; j < nb; ++j) {
            uint8_t* blk = dst + (n * nb + j) * 34;
            std::memcpy(blk, aux.data() + 2 * thq::q8t_d(n, nb, j), 2);
            std::memcpy(blk + 2, qs.data() + thq::q8t_q(n, nb, j, 0), 16);
            std::memcpy(blk + 18, qs.data() + thq::q8t_q(n, nb, j, 1), 16);
        }
    return THQ_OK;
}

int thq_dequantize(thq_ctx* ctx, const thq_weight* w, float* out_dev, void* stream) {
    if (!ctx || !w || !out_dev) return fail(THQ_EINVAL, "null argument");
    if (!aligned16(out_dev)) return fail(THQ_EALIGN, "out_dev must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = dequant_any(w, out_dev, false, s);
    if (e != hipSuccess) return fail(THQ_EHIP, "dequantize: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_dequantize_bf16(thq_ctx* ctx, const thq_weight* w, uint16_t* out_dev, void* stream) {
    if (!ctx || !w || !out_dev) return fail(THQ_EINVAL, "null argument");
    if (!aligned16(out_dev)) return fail(THQ_EALIGN, "out_dev must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    hipError_t e = dequant_any(w, out_dev, true, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(THQ_EHIP, "dequantize_bf16: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_affine_from_device(thq_ctx* ctx, const uint32_t* wq_dev, const uint16_t* sb_dev, int64_t n, int64_t k, int gs,
                           int tiled, void* stream, thq_weight** out) {
    if (!ctx || !wq_dev || !sb_dev || !out) return fail(THQ_EINVAL, "null argument");
    int rc = check_affine(n, k, gs, tiled);
    if (rc) return rc;
    if (((uintptr_t)wq_dev & 3u) || ((uintptr_t)sb_dev & 1u)) return fail(THQ_EALIGN, "wq/sb misaligned");
    DeviceGuard g(ctx->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    thq_weight* w = nullptr;
    rc = alloc_weight(ctx, THQ_MLX_Q4, n, k, &w);
    if (rc) return rc;
    w->gs = gs;
    hipError_t e = thq::launch_repack_affine(wq_dev, sb_dev, w->q, n, (int)k, gs, tiled != 0, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        thq_weight_free(w);
        return fail(THQ_EHIP, "affine repack: %s", hipGetErrorString(e));
    }
    *out = w;
    return THQ_OK;
}

int thq_affine_upload(thq_ctx* ctx, const uint32_t* wq_host, const uint16_t* sb_host, int64_t n, int64_t k, int gs,
                      int tiled, thq_weight** out) {
    if (!ctx || !wq_host || !sb_host || !out) return fail(THQ_EINVAL, "null argument");
    int rc = check_affine(n, k, gs, tiled);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    size_t wb, sbb;
    affine_src_bytes(n, k, gs, tiled, wb, sbb);
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, wb + sbb);
    if (e != hipSuccess) return fail(THQ_ENOMEM, "hipMalloc staging(%zu): %s", wb + sbb, hipGetErrorString(e));
    e = hipMemcpy(staging, wq_host, wb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(static_cast<char*>(staging) + wb, sb_host, sbb, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(staging);
        return fail(THQ_EHIP, "hipMemcpy affine weight: %s", hipGetErrorString(e));
    }
    rc = thq_affine_from_device(ctx, static_cast<const uint32_t*>(staging),
                                reinterpret_cast<const uint16_t*>(static_cast<char*>(staging) + wb), n, k, gs, tiled,
                                nullptr, out);  // synchronizes
    (void)hipFree(staging);
    return rc;
}

int thq_affine_download(const thq_weight* w, uint32_t* wq_host, uint16_t* sb_host) {
    if (!w || !wq_host || !sb_host) return fail(THQ_EINVAL, "null argument");
    if (w->qtype != THQ_MLX_Q4) return fail(THQ_EDTYPE, "not an MLX affine weight");
    DeviceGuard g(w->device);
    std::vector<uint8_t> qs(q_plane_bytes(w->qtype, w->N, w->K));
    HIP_TRY(hipMemcpy(qs.data(), w->q, qs.size(), hipMemcpyDeviceToHost));
    const int nsb = (int)((w->K + 255) / 256), ng = (int)(w->K / w->gs), per = w->gs / 64;
    const int64_t words = w->K / 8;
    for (int64_t n = 0; n < w->N; ++n) {
        for (int64_t gp = 0; gp < w->K / 64; ++gp) {
            const int s = (int)(gp >> 2), p = (int)(gp & 3);
            uint8_t pc[2][16];
            for (int h = 0; h < 2; ++h) std::memcpy(pc[h], qs.data() + thq::q4k_piece(n, nsb, s, h, p), 16);
            uint32_t* wd = wq_host + n * words + gp * 8;
            for (int i = 0; i < 8; ++i) wd[i] = 0;
            for (int h = 0; h < 2; ++h)
                for (int j = 0; j < 16; ++j) {
                    const uint32_t lo = pc[h][j] & 0xFu, hi = pc[h][j] >> 4;
                    wd[2 * h + (j >> 3)] |= lo << (4 * (j & 7));
                    wd[4 + 2 * h + (j >> 3)] |= hi << (4 * (j & 7));
                }
            if (gp % per == 0) {
                uint32_t hw;
                std::memcpy(&hw, qs.data() + thq::q4k_hdword(n, nsb, s, p), 4);
                sb_host[n * 2 * ng + gp / per] = (uint16_t)(hw & 0xFFFFu);
                sb_host[n * 2 * ng + ng + gp / per] = (uint16_t)(hw >> 16);
            }
        }
    }
    return THQ_OK;
}

int thq_quantize_act(thq_ctx* ctx, thq_dtype dot_type, const void* x_dev, thq_act x_type, int64_t m, int64_t k,
                     void* blocks_dev, void* stream) {
    if (!ctx) return fail(THQ_EINVAL, "null context");
    if (dot_type != THQ_Q8_0 && dot_type != THQ_Q8_K)
        return fail(THQ_EDTYPE, "dot type %d is not Q8_0 (8) or Q8_K (15)", (int)dot_type);
    if (x_type != THQ_ACT_F32 && x_type != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad x_type %d", (int)x_type);
    const int bs = dot_type == THQ_Q8_0 ? 32 : 256;
    if (m < 0 || k <= 0 || k % bs) return fail(THQ_ESHAPE, "shape [%lld, %lld] (K must be a positive multiple of %d)",
                                                (long long)m, (long long)k, bs);
    if (m == 0) return THQ_OK;
    if (!x_dev || !blocks_dev) return fail(THQ_EINVAL, "null argument");
    if (!aligned16(x_dev)) return fail(THQ_EALIGN, "x_dev must be 16-byte aligned");
    if ((uintptr_t)blocks_dev & (dot_type == THQ_Q8_0 ? 1u : 3u))
        return fail(THQ_EALIGN, "blocks_dev must be %d-byte aligned", dot_type == THQ_Q8_0 ? 2 : 4);
    DeviceGuard g(ctx->device);
    hipError_t e = thq::launch_quantize_act(dot_type == THQ_Q8_0 ? 8 : 12, x_dev, x_type == THQ_ACT_F32, m, k,
                                            blocks_dev, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(THQ_EHIP, "quantize_act: %s", hipGetErrorString(e));
    return THQ_OK;
}

size_t thq_q8act_bytes(thq_dtype dot_type, int64_t m, int64_t k) {
    if ((dot_type != THQ_Q8_0 && dot_type != THQ_Q8_K) || m < 0 || k <= 0) return 0;
    return thq::q8act_workspace_bytes(dot_type == THQ_Q8_0 ? 8 : 12, m, k);
}

int thq_q8act_prepare(thq_ctx* ctx, thq_dtype dot_type, const void* x_dev, thq_act x_type, int64_t m, int64_t k,
                      void* buf_dev, void* stream) {
    if (!ctx || !x_dev || !buf_dev) return fail(THQ_EINVAL, "null argument");
    if (dot_type != THQ_Q8_0 && dot_type != THQ_Q8_K) return fail(THQ_EDTYPE, "dot type %d (want Q8_0 or Q8_K)", dot_type);
    if (x_type != THQ_ACT_F32 && x_type != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad x_type %d", x_type);
    const int qt = dot_type == THQ_Q8_0 ? 8 : 12;
    const int bs = dot_type == THQ_Q8_0 ? 32 : 256;
    if (m < 0 || k <= 0 || k % bs) return fail(THQ_ESHAPE, "x [%lld, %lld]: K must be a positive multiple of %d",
                                               (long long)m, (long long)k, bs);
    if (!thq::q8act_supported(qt, k)) return fail(THQ_ESHAPE, "K=%lld too large for THQ_MODE_Q8ACT", (long long)k);
    if (!aligned16(x_dev)) return fail(THQ_EALIGN, "x_dev must be 16-byte aligned");
    if ((uintptr_t)buf_dev & 255u) return fail(THQ_EALIGN, "buf_dev must be 256-byte aligned");
    if (m == 0) return THQ_OK;
    DeviceGuard g(ctx->device);
    hipError_t e = thq::launch_q8act_prepare(qt, x_dev, x_type == THQ_ACT_F32, m, k, buf_dev,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(THQ_EHIP, "kernel launch: %s", hipGetErrorString(e));
    return THQ_OK;
}

namespace {

int run_q8act_dot(thq_ctx* ctx, const thq_weight* w, thq_dtype dot_type, const void* buf, int64_t m, int64_t k,
                  void* y, int yt, bool gu, void* stream) {
    if (!ctx || !w || !buf) return fail(THQ_EINVAL, "null argument");
    if (yt != THQ_ACT_F32 && yt != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad y_type %d", yt);
    if (w->qtype != THQ_Q8_0 && w->qtype != THQ_Q4_K)
        return fail(THQ_EDTYPE, "THQ_MODE_Q8ACT applies to Q8_0 and Q4_K weights");
    const thq_dtype want = w->qtype == THQ_Q8_0 ? THQ_Q8_0 : THQ_Q8_K;
    if (dot_type != want) return fail(THQ_EDTYPE, "buffer dot type %d, the weight's is %d", dot_type, want);
    if (k != w->K) return fail(THQ_ESHAPE, "buffer K=%lld, weight K=%lld", (long long)k, (long long)w->K);
    if (gu && (w->N % 2)) return fail(THQ_ESHAPE, "gate/up weight has an odd row count %lld", (long long)w->N);
    if (m < 0 || m > (1 << 24)) return fail(THQ_ESHAPE, "M=%lld out of range", (long long)m);
    if ((uintptr_t)buf & 255u) return fail(THQ_EALIGN, "buf_dev must be 256-byte aligned");
    if (m == 0) return THQ_OK;
    if (!y) return fail(THQ_EINVAL, "null y");
    DeviceGuard g(ctx->device);
    const int64_t nout = gu ? w->N / 2 : w->N;
    const thq::TilePlan tp = q8act_tile_plan(ctx, w, m, gu);
    hipError_t e;
    if (tp.kw > 0) {
        // the tile kernel; its K splits sum in the context workspace
        std::lock_guard<std::mutex> lk(ctx->mu);
        uint32_t* cnt = nullptr;
        if (tp.splits > 1) {
            const int rc = ensure_ws(ctx, tp.workspace_bytes);
            if (rc) return rc;
            if (tickets_on()) cnt = tile_counters(ctx, (w->N + 31) / 32);
        }
        e = thq::launch_q8act_dot_tile(tp, view(w), w->tq, buf, y, yt == THQ_ACT_F32, gu, (int)m,
                                       static_cast<float*>(ctx->ws), cnt, static_cast<hipStream_t>(stream));
    } else {
        e = thq::launch_q8act_dot(view(w), buf, y, yt == THQ_ACT_F32, gu, (int)m, nout, gu ? nout : 0,
                                  static_cast<hipStream_t>(stream));
    }
    if (e != hipSuccess) return fail(THQ_EHIP, "kernel launch: %s", hipGetErrorString(e));
    return THQ_OK;
}

}  // namespace

int thq_gate_up_silu_q8act_emit(thq_ctx* ctx, const thq_weight* fused, thq_dtype dot_type, const void* buf_dev,
                                int64_t m, int64_t k, void* y_dev, thq_act y_type, void* next_buf_dev, void* stream) {
    if (!ctx || !fused || !buf_dev || !next_buf_dev) return fail(THQ_EINVAL, "null argument");
    if (fused->qtype != THQ_Q4_K) return fail(THQ_EDTYPE, "the emitting gate/up takes Q4_K weights");
    if (fused->N % 512) return fail(THQ_ESHAPE, "gate/up outputs %lld: a multiple of 256 per half is needed",
                                    (long long)(fused->N / 2));
    if ((uintptr_t)next_buf_dev & 255u) return fail(THQ_EALIGN, "next_buf_dev must be 256-byte aligned");
    if ((uintptr_t)y_dev & 15u) return fail(THQ_EALIGN, "y_dev must be 16-byte aligned");
    const int64_t nout = fused->N / 2;
    if (!thq::q8act_supported(12, nout)) return fail(THQ_ESHAPE, "the next projection's K=%lld is too large",
                                                    (long long)nout);
    // the shared checks (dot type, K, y type, M) of the non-emitting call
    if (m < 0 || m > (1 << 24)) return fail(THQ_ESHAPE, "M=%lld out of range", (long long)m);
    if (dot_type != THQ_Q8_K) return fail(THQ_EDTYPE, "buffer dot type %d, the weight's is %d", dot_type, THQ_Q8_K);
    if (k != fused->K) return fail(THQ_ESHAPE, "buffer K=%lld, weight K=%lld", (long long)k, (long long)fused->K);
    if (y_type != THQ_ACT_F32 && y_type != THQ_ACT_BF16) return fail(THQ_EINVAL, "bad y_type %d", y_type);
    if ((uintptr_t)buf_dev & 255u) return fail(THQ_EALIGN, "buf_dev must be 256-byte aligned");
    if (m == 0) return THQ_OK;
    if (!y_dev) return fail(THQ_EINVAL, "null y");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::mutex> lk(ctx->mu);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const thq::TilePlan tp = q8act_tile_plan(ctx, fused, m, true);
    if (tp.kw > 0) {
        // a weight with a tile plane (2..8 rows): its int8 tile kernel, then
        // the next projection's planes quantized from y (the bytes
        // thq_q8act_prepare writes for y, by construction)
        uint32_t* cnt = nullptr;
        if (tp.splits > 1) {
            const int rc = ensure_ws(ctx, tp.workspace_bytes);
            if (rc) return rc;
            if (tickets_on()) cnt = tile_counters(ctx, (fused->N + 31) / 32);
        }
        hipError_t e = thq::launch_q8act_dot_tile(tp, view(fused), fused->tq, buf_dev, y_dev, y_type == THQ_ACT_F32,
                                                  true, (int)m, static_cast<float*>(ctx->ws), cnt, s);
        if (e == hipSuccess)
            e = thq::launch_q8act_prepare(12, y_dev, y_type == THQ_ACT_F32, m, nout, next_buf_dev, s);
        if (e != hipSuccess) return fail(THQ_EHIP, "kernel launch: %s", hipGetErrorString(e));
        return THQ_OK;
    }
    const size_t need = thq::q8act_emit_counters(m, fused->K, nout);
    if (need > ctx->emit_cnt_n) {
        // zeroed once here; every launch leaves them zero again
        size_t want = std::max(need + need / 8, 2 * ctx->emit_cnt_n);
        uint32_t* p = nullptr;
        hipError_t e = hipMalloc((void**)&p, want * sizeof(uint32_t));
        if (e == hipSuccess) e = hipMemset(p, 0, want * sizeof(uint32_t));
        if (e != hipSuccess) {
            if (p) (void)hipFree(p);
            return fail(THQ_ENOMEM, "emit counters (%zu): %s", want, hipGetErrorString(e));
        }
        if (ctx->emit_cnt) ctx->retired.push_back(ctx->emit_cnt);
        ctx->emit_cnt = p;
        ctx->emit_cnt_n = want;
    }
    hipError_t e = thq::launch_q8act_dot_emit(view(fused), buf_dev, y_dev, y_type == THQ_ACT_F32, (int)m, nout,
                                              ctx->emit_cnt, next_buf_dev, s);
    if (e != hipSuccess) return fail(THQ_EHIP, "kernel launch: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_matmul_q8act(thq_ctx* ctx, const thq_weight* w, thq_dtype dot_type, const void* buf_dev, int64_t m, int64_t k,
                     void* y_dev, thq_act y_type, void* stream) {
    return run_q8act_dot(ctx, w, dot_type, buf_dev, m, k, y_dev, y_type, false, stream);
}

int thq_gate_up_silu_q8act(thq_ctx* ctx, const thq_weight* fused, thq_dtype dot_type, const void* buf_dev, int64_t m,
                           int64_t k, void* y_dev, thq_act y_type, void* stream) {
    return run_q8act_dot(ctx, fused, dot_type, buf_dev, m, k, y_dev, y_type, true, stream);
}

int thq_matmul_noalloc(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m, void* y_dev,
                       thq_act y_type, uint32_t flags, void* stream) {
    // the kernels of thq_matmul on the device's static scratch: no hipMalloc,
    // hipFree or allocating library call; the partials each route writes
    // cover everything its reduce reads, so nothing needs clearing
    Call c{ctx, w, x_dev, x_type, m, y_dev, y_type, flags, false, static_cast<hipStream_t>(stream), nullptr};
    c.scratch_cap = THQ_NOALLOC_SCRATCH_BYTES;  // e.g. the dequantize-then-GEMM route falls back to the tile GEMM
    c.counters = false;                         // routes whose splits meet on arrival counters are not planned
    int rc = check_call(c);
    if (rc || m == 0) return rc;
    DeviceGuard g(ctx->device);
    const Route r = plan_route(c);
    if (r.scratch > THQ_NOALLOC_SCRATCH_BYTES)
        return fail(THQ_ESHAPE, "this call needs %zu bytes of scratch; thq_matmul_noalloc has %zu (use thq_matmul)",
                    r.scratch, THQ_NOALLOC_SCRATCH_BYTES);
    return exec_route(c, r, ctx->scratch);
}

size_t thq_noalloc_scratch_bytes(void) { return THQ_NOALLOC_SCRATCH_BYTES; }

int thq_call_scratch_bytes(thq_ctx* ctx, const thq_weight* w, int64_t m, thq_act x_type, uint32_t flags,
                           int gate_up, size_t* bytes) {
    if (!bytes) return fail(THQ_EINVAL, "null bytes");
    *bytes = 0;
    // the route depends on the operands' alignment only: plan with aligned
    // placeholders (nothing is dereferenced or launched)
    const uintptr_t ph = 256;
    Call c{ctx, w, reinterpret_cast<const void*>(ph), x_type, m, reinterpret_cast<void*>(ph), THQ_ACT_F32, flags,
           gate_up != 0, nullptr, nullptr};
    int rc = check_call(c);
    if (rc || m == 0) return rc;
    *bytes = plan_route(c).scratch;
    return THQ_OK;
}

int thq_reserve(thq_ctx* ctx, size_t workspace_bytes, int64_t counters) {
    if (!ctx) return fail(THQ_EINVAL, "null context");
    if (counters < 0 || counters > ((int64_t)1 << 32)) return fail(THQ_ESHAPE, "counters %lld out of range", (long long)counters);
    DeviceGuard g(ctx->device);
    std::lock_guard<std::mutex> lk(ctx->mu);
    int rc = ensure_ws(ctx, workspace_bytes);
    if (rc) return rc;
    if (counters > 0 && !tile_counters(ctx, counters))
        return fail(THQ_ENOMEM, "arrival counters (%lld entries) could not be allocated", (long long)counters);
    HIP_TRY(hipDeviceSynchronize());
    return THQ_OK;
}

size_t thq_workspace_bytes(const thq_ctx* ctx) {
    if (!ctx) return 0;
    std::lock_guard<std::mutex> lk(const_cast<thq_ctx*>(ctx)->mu);
    return ctx->ws_bytes;
}

int thq_matmul(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m, void* y_dev,
               thq_act y_type, uint32_t flags, void* stream) {
    return run_matmul(Call{ctx, w, x_dev, x_type, m, y_dev, y_type, flags, false, static_cast<hipStream_t>(stream),
                           nullptr});
}

int thq_gate_up_silu(thq_ctx* ctx, const thq_weight* fused, const void* x_dev, thq_act x_type, int64_t m, void* y_dev,
                     thq_act y_type, uint32_t flags, void* stream) {
    return run_matmul(Call{ctx, fused, x_dev, x_type, m, y_dev, y_type, flags, true, static_cast<hipStream_t>(stream),
                           nullptr});
}

int thq_argmax(thq_ctx* ctx, const float* v_dev, int64_t m, int64_t n, uint32_t* idx_dev, void* stream) {
    if (!ctx) return fail(THQ_EINVAL, "null context");
    if (m < 0 || n < 0) return fail(THQ_ESHAPE, "negative shape");
    if (m == 0) return THQ_OK;
    if (!idx_dev || (n > 0 && !v_dev)) return fail(THQ_EINVAL, "null argument");
    if (n > 0xFFFFFFFFll) return fail(THQ_ESHAPE, "row length exceeds u32 indices");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::mutex> lk(ctx->mu);
    int rc = ensure_ws(ctx, thq::argmax_workspace_bytes(m, n));
    if (rc) return rc;
    hipError_t e = thq::launch_argmax(v_dev, m, n, idx_dev, ctx->ws, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(THQ_EHIP, "argmax: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_topk(thq_ctx* ctx, const float* v_dev, int64_t m, int64_t n, int k, float* vals_dev, uint32_t* idx_dev,
             void* stream) {
    if (!ctx) return fail(THQ_EINVAL, "null context");
    if (k < 1 || k > 64) return fail(THQ_EINVAL, "k=%d (1..64)", k);
    if (m < 0 || n < 0) return fail(THQ_ESHAPE, "negative shape");
    if (n > 0xFFFFFFFFll) return fail(THQ_ESHAPE, "row length exceeds u32 indices");
    if (m == 0) return THQ_OK;
    if (!vals_dev || !idx_dev || (n > 0 && !v_dev)) return fail(THQ_EINVAL, "null argument");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::mutex> lk(ctx->mu);
    int rc = ensure_ws(ctx, thq::topk_workspace_bytes(m, n, k));
    if (rc) return rc;
    int64_t ncnt = 0;
    uint32_t* cnt = topk_counters(ctx, m, &ncnt);
    hipError_t e =
        thq::launch_topk(v_dev, m, n, k, vals_dev, idx_dev, ctx->ws, cnt, ncnt, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(THQ_EHIP, "topk: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_matmul_topk(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m, int k,
                    float* logits_dev, float* vals_dev, uint32_t* idx_dev, uint32_t flags, void* stream) {
    if (flags & ~(THQ_MODE_EXACT_W | THQ_MODE_Q8ACT)) return fail(THQ_EINVAL, "unknown flags 0x%x", flags);
    if (k < 1 || k > 64) return fail(THQ_EINVAL, "k=%d (1..64)", k);
    flags |= THQ_MODE_EXACT_W;
    hipStream_t s = static_cast<hipStream_t>(stream);
    Call c{ctx, w, x_dev, x_type, m, logits_dev ? static_cast<void*>(logits_dev) : static_cast<void*>(vals_dev),
           THQ_ACT_F32, flags, false, s, nullptr};
    int rc = check_call(c);
    if (rc || m == 0) return rc;
    if (!vals_dev || !idx_dev) return fail(THQ_EINVAL, "null vals_dev or idx_dev");
    if (w->N > 0xFFFFFFFFll) return fail(THQ_ESHAPE, "N=%lld exceeds u32 indices", (long long)w->N);
    DeviceGuard g(ctx->device);
    // logits (workspace head unless the caller gives a buffer), then the
    // route's scratch and the top-k candidates, reserved in one step
    const Route r = plan_route(c);
    const size_t lbytes = logits_dev ? 0 : round256((size_t)m * (size_t)w->N * sizeof(float));
    std::lock_guard<std::mutex> lk(ctx->mu);
    rc = ensure_ws(ctx, lbytes + std::max(r.scratch, thq::topk_workspace_bytes(m, w->N, k)));
    if (rc) return rc;
    float* logits = logits_dev ? logits_dev : static_cast<float*>(ctx->ws);
    void* scratch = static_cast<char*>(ctx->ws) + lbytes;
    c.y = logits;
    rc = exec_route(c, r, scratch);
    if (rc) return rc;
    int64_t ncnt = 0;
    uint32_t* cnt = topk_counters(ctx, m, &ncnt);
    hipError_t e = thq::launch_topk(logits, m, w->N, k, vals_dev, idx_dev, scratch, cnt, ncnt, s);
    if (e != hipSuccess) return fail(THQ_EHIP, "topk: %s", hipGetErrorString(e));
    return THQ_OK;
}

int thq_matmul_argmax(thq_ctx* ctx, const thq_weight* w, const void* x_dev, thq_act x_type, int64_t m,
                      float* logits_dev, uint32_t* idx_dev, uint32_t flags, void* stream) {
    if (flags & ~(THQ_MODE_EXACT_W | THQ_MODE_Q8ACT | THQ_MODE_ARGMAX_FUSED))
        return fail(THQ_EINVAL, "unknown flags 0x%x", flags);
    // no logits wanted and THQ_MODE_ARGMAX_FUSED: decode paths with the fused
    // epilogue write per-tile (max, index) partials instead of logits
    const bool fused = (flags & THQ_MODE_ARGMAX_FUSED) != 0;
    flags = (flags & ~THQ_MODE_ARGMAX_FUSED) | THQ_MODE_EXACT_W;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // validated as the logits-path call; without logits_dev, idx_dev stands in
    // for y until the logits are placed in the workspace
    Call c{ctx, w, x_dev, x_type, m, logits_dev ? static_cast<void*>(logits_dev) : static_cast<void*>(idx_dev),
           THQ_ACT_F32, flags, false, s, nullptr};
    int rc = check_call(c);
    if (rc || m == 0) return rc;
    if (!idx_dev) return fail(THQ_EINVAL, "null idx_dev");
    if (w->N > 0xFFFFFFFFll) return fail(THQ_ESHAPE, "N=%lld exceeds u32 indices", (long long)w->N);
    DeviceGuard g(ctx->device);
    thq::AmaxOut am;
    if (!logits_dev && fused && !(flags & THQ_MODE_Q8ACT) && (m <= 8 || (m >= 17 && m <= 64))) {
        c.am = &am;
        const Route r = plan_route(c);
        if (r.kind != Kind::NONE) {
            const int64_t ld = (w->N + 3) / 4;  // the most partials any fused path writes per row
            const size_t part = round256((size_t)m * (size_t)ld * 8);
            std::lock_guard<std::mutex> lk(ctx->mu);
            rc = ensure_ws(ctx, part + std::max(r.scratch, thq::argmax_partials_tmp_bytes(m, ld)));
            if (rc) return rc;
            am.v = static_cast<float*>(ctx->ws);
            am.i = reinterpret_cast<uint32_t*>(am.v + m * ld);
            am.ld = ld;
            am.nb = 0;
            rc = exec_route(c, r, static_cast<char*>(ctx->ws) + part);
            if (rc) return rc;
            if (am.nb > 0) {
                hipError_t e = thq::launch_argmax_partials(am.v, am.i, m, am.nb, ld, idx_dev,
                                                           static_cast<char*>(ctx->ws) + part, s);
                if (e != hipSuccess) return fail(THQ_EHIP, "argmax: %s", hipGetErrorString(e));
                return THQ_OK;
            }
            // this launch path has no fused epilogue after all: nothing ran
        }
    }
    // logits path.  Without logits_dev the logits take the workspace head and
    // the route's scratch (split-K partials, quantized activations) and the
    // argmax scratch follow them: one reservation, sized from the route the
    // call will take, before any pointer into the workspace is formed
    c.am = nullptr;
    const Route r = plan_route(c);
    const size_t lbytes = logits_dev ? 0 : round256((size_t)m * (size_t)w->N * sizeof(float));
    std::lock_guard<std::mutex> lk(ctx->mu);
    rc = ensure_ws(ctx, lbytes + std::max(r.scratch, thq::argmax_workspace_bytes(m, w->N)));
    if (rc) return rc;
    float* logits = logits_dev ? logits_dev : static_cast<float*>(ctx->ws);
    void* scratch = static_cast<char*>(ctx->ws) + lbytes;
    c.y = logits;
    rc = exec_route(c, r, scratch);
    if (rc) return rc;
    hipError_t e = thq::launch_argmax(logits, m, w->N, idx_dev, scratch, s);
    if (e != hipSuccess) return fail(THQ_EHIP, "argmax: %s", hipGetErrorString(e));
    return THQ_OK;
}

namespace {
int kernel_qtype(int dtype) {
    switch (dtype) {
        case THQ_Q8_0: return 8;
        case THQ_Q4_K: return 12;
        case THQ_Q6_K: return 14;
        case THQ_MLX_Q4: return 13;
        default: return 0;
    }
}
}  // namespace

int thq_plan_gemv_mfma(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, thq_gemv_plan_info* out) {
    const int qt = kernel_qtype(dtype);
    if (!qt) return fail(THQ_EDTYPE, "dtype %d", dtype);
    if (!out) return fail(THQ_EINVAL, "null out");
    if (m < 1 || n < 1 || k < 1) return fail(THQ_ESHAPE, "shape [%lld, %lld, %lld]", (long long)m, (long long)n,
                                             (long long)k);
    const thq::GemvPlan p = thq::plan_gemv_mfma(qt, m, n, k, gate_up != 0);
    const thq::GemvInstance in = thq::gemv_mfma_instance(qt, (int)std::min<int64_t>(m, 1 << 20), p);
    const thq::GemvLimits l = thq::gemv_mfma_limits();
    *out = thq_gemv_plan_info{};
    out->waves = p.waves;
    out->chunks_per_wave = p.cpw;
    out->splits = p.splits;
    out->live_rows = in.E;
    out->staged_per_thread = in.NX;
    out->workspace_bytes = (int64_t)p.workspace_bytes;
    out->xs_elems = l.xs_elems;
    out->xs_pad_elems = l.xs_pad_elems;
    out->kb_max = l.kb_max;
    out->kb_max_e8 = l.kb_max_e8;
    out->mmax = l.mmax;
    out->max_waves = l.max_waves;
    out->sums_rows_e4 = l.sums_rows_e4;
    out->sums_cols_e4 = l.sums_cols_e4;
    out->sums_rows_e8 = l.sums_rows_e8;
    out->sums_cols_e8 = l.sums_cols_e8;
    return THQ_OK;
}

int thq_plan_gemv_wide(int dtype, int64_t m, int64_t n, int64_t k, int cus, thq_wide_plan_info* out) {
    const int qt = kernel_qtype(dtype);
    if (!qt) return fail(THQ_EDTYPE, "dtype %d", dtype);
    if (!out) return fail(THQ_EINVAL, "null out");
    if (m < 1 || n < 1 || k < 1) return fail(THQ_ESHAPE, "shape [%lld, %lld, %lld]", (long long)m, (long long)n,
                                             (long long)k);
    const thq::WidePlan p = thq::plan_gemv_wide(qt, m, n, k, cus);
    *out = thq_wide_plan_info{};
    out->splits = p.splits;
    out->chunks_per_split = p.cps;
    out->workspace_bytes = (int64_t)p.workspace_bytes;
    return THQ_OK;
}

int thq_plan_gemm_mid(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, int cus, thq_mid_plan_info* out) {
    if (dtype != THQ_Q4_K && dtype != THQ_MLX_Q4)
        return fail(THQ_EDTYPE, "the streaming GEMM: Q4_K or MLX affine (%d)", dtype);
    if (!out) return fail(THQ_EINVAL, "null out");
    if (m < 1 || n < 1 || k < 1) return fail(THQ_ESHAPE, "shape [%lld, %lld, %lld]", (long long)m, (long long)n,
                                             (long long)k);
    const thq::MidPlan p = thq::plan_gemm_mid(kernel_qtype(dtype), m, n, k, gate_up != 0, cus);
    *out = thq_mid_plan_info{};
    out->group_halves = p.mh;
    out->col_tiles = p.nt;
    out->waves = p.nw;
    out->groups = p.groups;
    out->splits = p.splits;
    out->chunks_per_split = p.cps;
    out->workspace_bytes = (int64_t)p.workspace_bytes;
    return THQ_OK;
}

int thq_plan_gemv_tile(int dtype, int64_t m, int64_t n, int64_t k, int gate_up, int cus,
                       thq_tile_plan_info* out) {
    if (dtype != THQ_Q4_K && dtype != THQ_MLX_Q4) return fail(THQ_EDTYPE, "tile planes: Q4_K or MLX affine (%d)", dtype);
    if (!out) return fail(THQ_EINVAL, "null out");
    if (m < 1 || n < 1 || k < 1) return fail(THQ_ESHAPE, "shape [%lld, %lld, %lld]", (long long)m, (long long)n,
                                             (long long)k);
    const thq::TilePlan p = thq::plan_gemv_tile(m, n, k, gate_up != 0, cus);
    *out = thq_tile_plan_info{};
    out->waves = p.kw;
    out->splits = p.splits;
    out->workspace_bytes = (int64_t)p.workspace_bytes;
    return THQ_OK;
}

int thq_plan_gemm(int dtype, int exact, int64_t m, int64_t n, int64_t k, int gate_up, int cus,
                  thq_gemm_plan_info* out) {
    const int qt = kernel_qtype(dtype);
    if (!qt) return fail(THQ_EDTYPE, "dtype %d", dtype);
    if (!out) return fail(THQ_EINVAL, "null out");
    if (m < 1 || n < 1 || k < 1) return fail(THQ_ESHAPE, "shape [%lld, %lld, %lld]", (long long)m, (long long)n,
                                             (long long)k);
    const thq::GemmPlan p = thq::plan_gemm(qt, exact != 0, m, n, k, gate_up != 0, cus);
    *out = thq_gemm_plan_info{};
    out->bm = p.bm;
    out->splits = p.splits;
    out->k_steps = p.kps;
    out->tiles_n = p.tiles_n;
    out->tiles_m = p.tiles_m;
    out->workspace_bytes = (int64_t)p.workspace_bytes;
    return THQ_OK;
}

}  // extern "C"
