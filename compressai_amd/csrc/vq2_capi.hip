// vq2_capi.hip -- the extern "C" boundary of libvq2_amd.so.
//
// Every entry validates its arguments on the host (pointers, dtypes, sizes,
// alignment) and returns a status code; nothing here allocates, synchronises
// or aborts.  Reference interfaces are cited in include/vq2_amd.h.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "vq2_internal.hpp"

namespace vq2 {

static thread_local char g_err[512] = {0};

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int set_hip_error(hipError_t err, const char* what)
{
    snprintf(g_err, sizeof(g_err), "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
    return VQ2_ERR_HIP;
}

void clear_error() { g_err[0] = 0; }

int device_cu_count()
{
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
        cache[dev] = cu;
    }
    return cache[dev];
}

}  // namespace vq2

using namespace vq2;

#define CHECK(cond, ...)                                    \
    do {                                                    \
        if (!(cond)) return set_error(VQ2_ERR_ARG, __VA_ARGS__); \
    } while (0)

static int check_codebooks(int s2, const void* cb0, const void* cb1, int cb_dt)
{
    CHECK(dt_ok(cb_dt), "codebook dtype %d invalid", cb_dt);
    CHECK(cb0 != nullptr, "cb0 is NULL");
    CHECK((uintptr_t)cb0 % 16 == 0, "cb0 must be 16-byte aligned");
    CHECK(s2 == VQ2_S2_NONE || s2 == VQ2_S2_U8 || s2 == VQ2_S2_U16, "s2_kind %d invalid", s2);
    if (s2 != VQ2_S2_NONE) {
        CHECK(cb1 != nullptr, "cb1 is NULL for a two-stage matrix");
        CHECK((uintptr_t)cb1 % 16 == 0, "cb1 must be 16-byte aligned");
    }
    return VQ2_OK;
}

extern "C" {

int vq2_version(void) { return 100; }

const char* vq2_last_error(void) { return g_err; }

// The fused-rotation entries read perm / sign with vector loads.
static int check_rot_tables(const int32_t* perm, const int8_t* sign)
{
    CHECK((uintptr_t)perm % 16 == 0, "perm must be 16-byte aligned");
    CHECK((uintptr_t)sign % 8 == 0, "sign must be 8-byte aligned");
    return VQ2_OK;
}

static GemvCall base_call(const void* x, int x_dt, int s2, const void* cb0, const void* cb1, int cb_dt, int s_dt,
                          int y_dt, int64_t ng, int64_t batch, float rs, void* stream)
{
    GemvCall c{};
    c.x = x;
    c.x_dt = x_dt;
    c.x_pdiv = 1;
    c.s2 = s2;
    c.cb0 = cb0;
    c.cb1 = cb1;
    c.cb_dt = cb_dt;
    c.s_dt = s_dt;
    c.n_experts = 1;
    c.P = 1;
    c.n_out_groups = 1;
    c.y_dt = y_dt;
    c.ng = ng;
    c.batch = batch;
    c.rs = rs;
    c.stream = stream;
    c.xscale = 1.0f;
    return c;
}

int vq2_gemv(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int16_t* idx0, const void* idx1,
             int s2_kind, const void* cb0, const void* cb1, int cb_dt, const void* scale, int s_dt, void* y, int y_dt,
             int64_t y_stride, int64_t out_rows, int64_t n, float rs, void* stream)
{
    clear_error();
    CHECK(batch >= 0 && out_rows >= 0 && n > 0, "vq2_gemv: bad sizes batch=%lld out_rows=%lld n=%lld", (long long)batch,
          (long long)out_rows, (long long)n);
    CHECK(n % 8 == 0, "vq2_gemv: n=%lld is not a multiple of 8", (long long)n);
    if (batch == 0 || out_rows == 0) return VQ2_OK;
    CHECK(x && idx0 && scale && y, "vq2_gemv: NULL pointer argument");
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(y_dt), "vq2_gemv: bad dtype code");
    CHECK(x_stride >= n && y_stride >= out_rows, "vq2_gemv: strides too small");
    int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
    if (r) return r;
    CHECK((s2_kind == VQ2_S2_NONE) == (idx1 == nullptr), "vq2_gemv: idx1 must be given iff s2_kind != NONE");
    GemvCall c = base_call(x, x_dt, s2_kind, cb0, cb1, cb_dt, s_dt, y_dt, n / 8, batch, rs, stream);
    c.x_bstride = x_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{idx0, idx1, scale, y, out_rows, y_stride};
    return gemv_launch(c);
}

size_t vq2_gemm_small_m_workspace(int64_t batch, int64_t out_rows, int64_t n)
{
    if (batch < 1 || batch > 64 || out_rows < 1 || n < 64 || n % 64) return 0;
    return gemm_small_m_workspace_bytes(batch, out_rows, n / 8);
}

// Validates a small-M GEMM call and fills `c`; returns VQ2_OK, an error, or
// -1 for an empty problem (nothing to launch).
static int small_m_call(GemmCall& c, const char* who, const void* x, int x_dt, int64_t batch, int64_t x_stride,
                        const int16_t* idx0, const void* idx1, int s2_kind, const void* cb0, const void* cb1,
                        int cb_dt, const void* scale, int s_dt, void* y, int y_dt, int64_t y_stride,
                        int64_t out_rows, int64_t n, float rs, void* stream)
{
    CHECK(batch >= 0 && batch <= 64 && out_rows >= 0 && n > 0, "%s: bad sizes batch=%lld (0..64) out_rows=%lld n=%lld",
          who, (long long)batch, (long long)out_rows, (long long)n);
    CHECK(n % 64 == 0, "%s: n=%lld is not a multiple of 64", who, (long long)n);
    if (batch == 0 || out_rows == 0) return -1;
    CHECK(x && idx0 && scale && y, "%s: NULL pointer argument", who);
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(y_dt), "%s: bad dtype code", who);
    CHECK(x_stride >= n && y_stride >= out_rows, "%s: strides too small", who);
    int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
    if (r) return r;
    CHECK((s2_kind == VQ2_S2_NONE) == (idx1 == nullptr), "%s: idx1 must be given iff s2_kind != NONE", who);
    c = GemmCall{};
    c.x = x;
    c.x_dt = x_dt;
    c.x_stride = x_stride;
    c.m = batch;
    c.idx0 = idx0;
    c.idx1 = idx1;
    c.s2 = s2_kind;
    c.cb0 = cb0;
    c.cb1 = cb1;
    c.cb_dt = cb_dt;
    c.scale = scale;
    c.s_dt = s_dt;
    c.y = y;
    c.y_dt = y_dt;
    c.y_stride = y_stride;
    c.out_rows = out_rows;
    c.ng = n / 8;
    c.rs = rs;
    c.stream = stream;
    return VQ2_OK;
}

int vq2_gemm_small_m(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int16_t* idx0, const void* idx1,
                     int s2_kind, const void* cb0, const void* cb1, int cb_dt, const void* scale, int s_dt, void* y,
                     int y_dt, int64_t y_stride, int64_t out_rows, int64_t n, float rs, void* workspace,
                     size_t ws_bytes, void* stream)
{
    clear_error();
    GemmCall c;
    const int r = small_m_call(c, "vq2_gemm_small_m", x, x_dt, batch, x_stride, idx0, idx1, s2_kind, cb0, cb1, cb_dt,
                               scale, s_dt, y, y_dt, y_stride, out_rows, n, rs, stream);
    if (r) return r < 0 ? VQ2_OK : r;
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    return gemm_small_m_launch(c);
}

int vq2_gemm_small_m_noalloc(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int16_t* idx0,
                             const void* idx1, int s2_kind, const void* cb0, const void* cb1, int cb_dt,
                             const void* scale, int s_dt, void* y, int y_dt, int64_t y_stride, int64_t out_rows,
                             int64_t n, float rs, void* stream)
{
    clear_error();
    GemmCall c;
    const int r = small_m_call(c, "vq2_gemm_small_m_noalloc", x, x_dt, batch, x_stride, idx0, idx1, s2_kind, cb0,
                               cb1, cb_dt, scale, s_dt, y, y_dt, y_stride, out_rows, n, rs, stream);
    if (r) return r < 0 ? VQ2_OK : r;
    return gemm_small_m_noalloc_launch(c);
}

size_t vq2_gemm_small_m_argmax_workspace(int64_t batch, int64_t out_rows, int64_t n)
{
    if (batch < 1 || batch > 64 || out_rows < 1 || n < 64 || n % 64) return 0;
    return gemm_small_m_top1_workspace_bytes(batch, out_rows, n / 8);
}

int vq2_gemm_small_m_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int16_t* idx0,
                            const void* idx1, int s2_kind, const void* cb0, const void* cb1, int cb_dt,
                            const void* scale, int s_dt, int64_t out_rows, int64_t n, float rs, void* workspace,
                            size_t ws_bytes, int64_t* out_idx, float* out_val, void* stream)
{
    clear_error();
    CHECK(batch >= 0 && batch <= 64 && out_rows >= 1 && out_rows <= 0xFFFFFFFFLL && n > 0,
          "vq2_gemm_small_m_argmax: bad sizes batch=%lld (0..64) out_rows=%lld n=%lld", (long long)batch,
          (long long)out_rows, (long long)n);
    CHECK(n % 64 == 0, "vq2_gemm_small_m_argmax: n=%lld is not a multiple of 64", (long long)n);
    if (batch == 0) return VQ2_OK;
    CHECK(x && idx0 && scale && out_idx, "vq2_gemm_small_m_argmax: NULL pointer argument");
    CHECK((uintptr_t)out_idx % 8 == 0, "vq2_gemm_small_m_argmax: out_idx must be 8-byte aligned");
    CHECK(dt_ok(x_dt) && dt_ok(s_dt), "vq2_gemm_small_m_argmax: bad dtype code");
    CHECK(x_stride >= n, "vq2_gemm_small_m_argmax: x_stride < n");
    int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
    if (r) return r;
    CHECK((s2_kind == VQ2_S2_NONE) == (idx1 == nullptr),
          "vq2_gemm_small_m_argmax: idx1 must be given iff s2_kind != NONE");
    GemmCall c{};
    c.x = x;
    c.x_dt = x_dt;
    c.x_stride = x_stride;
    c.m = batch;
    c.idx0 = idx0;
    c.idx1 = idx1;
    c.s2 = s2_kind;
    c.cb0 = cb0;
    c.cb1 = cb1;
    c.cb_dt = cb_dt;
    c.scale = scale;
    c.s_dt = s_dt;
    c.y_dt = VQ2_DT_F32;
    c.out_rows = out_rows;
    c.ng = n / 8;
    c.rs = rs;
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    c.stream = stream;
    return gemm_small_m_top1_launch(c, out_idx, out_val);
}

int vq2_gemv_rht(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int32_t* perm, const int8_t* sign,
                 int64_t hb, float rht_scale, int n_seg, const vq2_seg* segs, int s2_kind, const void* cb0,
                 const void* cb1, int cb_dt, int s_dt, int y_dt, int64_t n, float rs, void* stream)
{
    clear_error();
    CHECK(batch >= 0 && n > 0 && n % 8 == 0, "vq2_gemv_rht: bad sizes");
    CHECK(n_seg >= 1 && n_seg <= 4 && segs, "vq2_gemv_rht: 1..4 segments required");
    if (batch == 0) return VQ2_OK;
    CHECK(x, "vq2_gemv_rht: NULL activation");
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(y_dt), "vq2_gemv_rht: bad dtype code");
    CHECK(x_stride >= n, "vq2_gemv_rht: x_stride < n");
    CHECK(hb == 0 || (hb >= 2 && hb <= 8192 && (hb & (hb - 1)) == 0 && n % hb == 0),
          "vq2_gemv_rht: hb=%lld must be 0 (x already rotated) or a power of two in [2, 8192] dividing n",
          (long long)hb);
    if (hb)
        if (int rr = check_rot_tables(perm, sign)) return rr;
    int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
    if (r) return r;
    GemvCall c = base_call(x, x_dt, s2_kind, cb0, cb1, cb_dt, s_dt, y_dt, n / 8, batch, rs, stream);
    c.x_bstride = x_stride;
    c.nseg = n_seg;
    for (int s = 0; s < n_seg; s++) {
        const vq2_seg& g = segs[s];
        CHECK(g.out_rows >= 0, "vq2_gemv_rht: segment %d has negative rows", s);
        CHECK(g.out_rows == 0 || (g.idx0 && g.scale && g.y), "vq2_gemv_rht: segment %d has a NULL pointer", s);
        CHECK((s2_kind == VQ2_S2_NONE) == (g.idx1 == nullptr), "vq2_gemv_rht: segment %d idx1 mismatch", s);
        CHECK(g.y_stride >= g.out_rows, "vq2_gemv_rht: segment %d y_stride < out_rows", s);
        c.seg[s] = GemvSegCall{g.idx0, g.idx1, g.scale, g.y, g.out_rows, g.y_stride};
    }
    c.xm = hb ? 1 : 0;
    c.perm = perm;
    c.sign = sign;
    c.hb = hb;
    c.xscale = hb ? rht_scale : 1.0f;
    return gemv_launch(c);
}

int vq2_moe_grouped(const void* x, int x_dt, int64_t x_pair_stride, int64_t pairs_per_x, const void* ids,
                    int ids_dt, int64_t n_pairs, const int16_t* pool, int64_t n_experts, const void* cb, int cb_dt,
                    const void* pool_scale, int s_dt, void* y, int y_dt, int64_t y_pair_stride, int64_t out_rows,
                    int64_t ng, float rs, void* stream)
{
    clear_error();
    CHECK(n_pairs >= 0 && out_rows >= 0 && ng > 0 && n_experts > 0, "vq2_moe_grouped: bad sizes");
    if (n_pairs == 0 || out_rows == 0) return VQ2_OK;
    CHECK(x && ids && pool && pool_scale && y, "vq2_moe_grouped: NULL pointer argument");
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(y_dt), "vq2_moe_grouped: bad dtype code");
    CHECK(ids_dt == VQ2_ID_I32 || ids_dt == VQ2_ID_I64, "vq2_moe_grouped: bad ids dtype");
    CHECK(x_pair_stride == 0 || x_pair_stride >= ng * 8, "vq2_moe_grouped: x_pair_stride must be 0 or >= n");
    CHECK(pairs_per_x >= 1 && pairs_per_x <= 0x7FFFFFFF, "vq2_moe_grouped: pairs_per_x must be >= 1");
    CHECK(y_pair_stride >= out_rows, "vq2_moe_grouped: y_pair_stride < out_rows");
    CHECK(n_pairs <= 65535, "vq2_moe_grouped: n_pairs=%lld > 65535", (long long)n_pairs);
    int r = check_codebooks(VQ2_S2_NONE, cb, nullptr, cb_dt);
    if (r) return r;
    GemvCall c = base_call(x, x_dt, VQ2_S2_NONE, cb, nullptr, cb_dt, s_dt, y_dt, ng, 1, rs, stream);
    c.x_bstride = ng * 8;
    c.x_pstride = x_pair_stride;
    c.x_pdiv = (int)pairs_per_x;
    c.ids = ids;
    c.ids_i64 = ids_dt == VQ2_ID_I64;
    c.n_experts = n_experts;
    c.n_out_groups = n_pairs;
    c.y_ostride = y_pair_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{pool, nullptr, pool_scale, y, out_rows, 0};
    return gemv_launch(c);
}

// Grouped gate_up with the RHT prologue; pool1 / cb1 give the uint8 stage-2
// plane of (16,8) experts (s2 VQ2_S2_U8), else s2 is VQ2_S2_NONE.
static int moe_gate_up_rht(const char* fn, const void* h, int h_dt, int64_t tokens, const int32_t* perm,
                           const int8_t* sign, int64_t hb, float rht_scale, const void* ids, int ids_dt, int64_t P,
                           const int16_t* pool, const uint8_t* pool1, int s2, int64_t n_experts, const void* cb,
                           const void* cb1, int cb_dt, const void* pool_scale, int s_dt, void* y, int y_dt,
                           int64_t y_pair_stride, int64_t out_rows, int64_t ng, float rs, void* stream)
{
    clear_error();
    CHECK(tokens >= 0 && P > 0 && out_rows >= 0 && ng > 0 && n_experts > 0, "%s: bad sizes", fn);
    if (tokens == 0 || out_rows == 0) return VQ2_OK;
    CHECK(h && ids && pool && pool_scale && y, "%s: NULL pointer argument", fn);
    CHECK(s2 == VQ2_S2_NONE || pool1, "%s: NULL stage-2 plane", fn);
    CHECK(dt_ok(h_dt) && dt_ok(s_dt) && dt_ok(y_dt), "%s: bad dtype code", fn);
    CHECK(ids_dt == VQ2_ID_I32 || ids_dt == VQ2_ID_I64, "%s: bad ids dtype", fn);
    CHECK(y_pair_stride >= out_rows, "%s: y_pair_stride < out_rows", fn);
    CHECK(tokens * P <= 65535, "%s: too many pairs", fn);
    CHECK(hb >= 2 && hb <= 8192 && (hb & (hb - 1)) == 0 && (ng * 8) % hb == 0, "%s: bad hb", fn);
    if (int rr = check_rot_tables(perm, sign)) return rr;
    int r = check_codebooks(s2, cb, cb1, cb_dt);
    if (r) return r;
    GemvCall c = base_call(h, h_dt, s2, cb, cb1, cb_dt, s_dt, y_dt, ng, 1, rs, stream);
    c.x_bstride = ng * 8;
    c.x_pstride = ng * 8;
    c.x_pdiv = (int)P;
    c.ids = ids;
    c.ids_i64 = ids_dt == VQ2_ID_I64;
    c.n_experts = n_experts;
    c.n_out_groups = tokens * P;
    c.y_ostride = y_pair_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{pool, pool1, pool_scale, y, out_rows, 0};
    c.xm = 1;
    c.perm = perm;
    c.sign = sign;
    c.hb = hb;
    c.xscale = rht_scale;
    return gemv_launch(c);
}

int vq2_moe_gate_up_rht(const void* h, int h_dt, int64_t tokens, const int32_t* perm, const int8_t* sign, int64_t hb,
                        float rht_scale, const void* ids, int ids_dt, int64_t P, const int16_t* pool,
                        int64_t n_experts, const void* cb, int cb_dt, const void* pool_scale, int s_dt, void* y,
                        int y_dt, int64_t y_pair_stride, int64_t out_rows, int64_t ng, float rs, void* stream)
{
    return moe_gate_up_rht("vq2_moe_gate_up_rht", h, h_dt, tokens, perm, sign, hb, rht_scale, ids, ids_dt, P, pool,
                           nullptr, VQ2_S2_NONE, n_experts, cb, nullptr, cb_dt, pool_scale, s_dt, y, y_dt,
                           y_pair_stride, out_rows, ng, rs, stream);
}

int vq2_moe_gate_up_rht_16_8(const void* h, int h_dt, int64_t tokens, const int32_t* perm, const int8_t* sign,
                             int64_t hb, float rht_scale, const void* ids, int ids_dt, int64_t P, const int16_t* pool,
                             const uint8_t* pool1, int64_t n_experts, const void* cb, const void* cb1, int cb_dt,
                             const void* pool_scale, int s_dt, void* y, int y_dt, int64_t y_pair_stride,
                             int64_t out_rows, int64_t ng, float rs, void* stream)
{
    return moe_gate_up_rht("vq2_moe_gate_up_rht_16_8", h, h_dt, tokens, perm, sign, hb, rht_scale, ids, ids_dt, P,
                           pool, pool1, VQ2_S2_U8, n_experts, cb, cb1, cb_dt, pool_scale, s_dt, y, y_dt,
                           y_pair_stride, out_rows, ng, rs, stream);
}

int vq2_moe_router_gate_up_rht(const void* h, int h_dt, int64_t tokens, const int32_t* perm, const int8_t* sign,
                               int64_t hb, float rht_scale, const void* logits, int l_dt, int64_t n_routed, int k,
                               const void* shared_gate, int g_dt, int64_t shared_id, const int16_t* pool,
                               int64_t n_experts, const void* cb, int cb_dt, const void* pool_scale, int s_dt, void* y,
                               int y_dt, int64_t y_pair_stride, int64_t out_rows, int64_t ng, float rs, int32_t* ids,
                               float* w, void* stream)
{
    clear_error();
    CHECK(tokens >= 0 && out_rows >= 0 && ng > 0 && n_experts > 0, "vq2_moe_router_gate_up_rht: bad sizes");
    CHECK(n_routed >= 1 && n_routed <= 1024, "vq2_moe_router_gate_up_rht: n_routed=%lld not in [1, 1024]",
          (long long)n_routed);
    CHECK(k >= 1 && k <= 32 && k <= n_routed, "vq2_moe_router_gate_up_rht: k=%d out of range", k);
    CHECK(n_routed <= n_experts, "vq2_moe_router_gate_up_rht: the pool holds %lld experts < n_routed=%lld",
          (long long)n_experts, (long long)n_routed);
    CHECK(shared_id < n_experts, "vq2_moe_router_gate_up_rht: shared_id=%lld outside the pool", (long long)shared_id);
    if (tokens == 0 || out_rows == 0) return VQ2_OK;
    CHECK(h && logits && pool && pool_scale && y && ids && w, "vq2_moe_router_gate_up_rht: NULL pointer argument");
    CHECK(dt_ok(h_dt) && dt_ok(l_dt) && dt_ok(s_dt) && dt_ok(y_dt), "vq2_moe_router_gate_up_rht: bad dtype code");
    if (shared_id >= 0) CHECK(shared_gate && dt_ok(g_dt), "vq2_moe_router_gate_up_rht: the shared expert needs its gate");
    const int64_t P = k + (shared_id >= 0 ? 1 : 0);
    CHECK(y_pair_stride >= out_rows, "vq2_moe_router_gate_up_rht: y_pair_stride < out_rows");
    CHECK(tokens * P <= 65535, "vq2_moe_router_gate_up_rht: too many pairs");
    CHECK(hb >= 2 && hb <= 8192 && (hb & (hb - 1)) == 0 && (ng * 8) % hb == 0, "vq2_moe_router_gate_up_rht: bad hb");
    if (int rr = check_rot_tables(perm, sign)) return rr;
    int r = check_codebooks(VQ2_S2_NONE, cb, nullptr, cb_dt);
    if (r) return r;
    GemvCall c = base_call(h, h_dt, VQ2_S2_NONE, cb, nullptr, cb_dt, s_dt, y_dt, ng, 1, rs, stream);
    c.x_bstride = ng * 8;
    c.x_pstride = ng * 8;
    c.x_pdiv = (int)P;
    c.ids = ids;
    c.ids_i64 = 0;
    c.n_experts = n_experts;
    c.n_out_groups = tokens * P;
    c.y_ostride = y_pair_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{pool, nullptr, pool_scale, y, out_rows, 0};
    c.xm = 3;
    c.perm = perm;
    c.sign = sign;
    c.hb = hb;
    c.xscale = rht_scale;
    c.r_logits = logits;
    c.r_ldt = l_dt;
    c.r_ne = n_routed;
    c.r_k = k;
    c.r_pairs = (int)P;
    c.r_shared = shared_id;
    c.r_gate = shared_gate;
    c.r_gdt = g_dt;
    c.r_ids = ids;
    c.r_w = w;
    return gemv_launch(c);
}

int vq2_moe_down_combine(const void* x, int x_dt, const void* ids, int ids_dt, const float* w, int64_t tokens,
                         int64_t P, const int16_t* pool, int64_t n_experts, const void* cb, int cb_dt,
                         const void* pool_scale, int s_dt, void* out, int out_dt, int64_t out_stride,
                         int64_t out_rows, int64_t ng, float rs, void* stream)
{
    clear_error();
    CHECK(tokens >= 0 && P > 0 && out_rows >= 0 && ng > 0 && n_experts > 0, "vq2_moe_down_combine: bad sizes");
    if (tokens == 0 || out_rows == 0) return VQ2_OK;
    CHECK(x && ids && w && pool && pool_scale && out, "vq2_moe_down_combine: NULL pointer argument");
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(out_dt), "vq2_moe_down_combine: bad dtype code");
    CHECK(ids_dt == VQ2_ID_I32 || ids_dt == VQ2_ID_I64, "vq2_moe_down_combine: bad ids dtype");
    CHECK(out_stride >= out_rows, "vq2_moe_down_combine: out_stride < out_rows");
    CHECK(tokens <= 65535 && P <= 4096, "vq2_moe_down_combine: too many tokens/pairs");
    int r = check_codebooks(VQ2_S2_NONE, cb, nullptr, cb_dt);
    if (r) return r;
    GemvCall c = base_call(x, x_dt, VQ2_S2_NONE, cb, nullptr, cb_dt, s_dt, out_dt, ng, 1, rs, stream);
    c.x_bstride = ng * 8;
    c.x_pstride = ng * 8;
    c.ids = ids;
    c.ids_i64 = ids_dt == VQ2_ID_I64;
    c.n_experts = n_experts;
    c.pair_w = w;
    c.P = (int)P;
    c.n_out_groups = tokens;
    c.y_ostride = out_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{pool, nullptr, pool_scale, out, out_rows, 0};
    return gemv_launch(c);
}

// SwiGLU + RHT + grouped down + weighted combine; s2 / pool1 / cb1 as in
// moe_gate_up_rht; accumulate: out += the combine instead of out = it.
static int moe_down_swiglu_combine(const char* fn, const void* gu, int gu_dt, int64_t gu_stride,
                                   const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                                   const void* ids, int ids_dt, const float* w, int64_t tokens, int64_t P,
                                   const int16_t* pool, const uint8_t* pool1, int s2, int64_t n_experts,
                                   const void* cb, const void* cb1, int cb_dt, const void* pool_scale, int s_dt,
                                   void* out, int out_dt, int64_t out_stride, int64_t out_rows, int64_t ng, float rs,
                                   int accumulate, void* stream)
{
    clear_error();
    CHECK(tokens >= 0 && P > 0 && out_rows >= 0 && ng > 0 && n_experts > 0, "%s: bad sizes", fn);
    if (tokens == 0 || out_rows == 0) return VQ2_OK;
    CHECK(gu && ids && w && pool && pool_scale && out, "%s: NULL pointer argument", fn);
    CHECK(s2 == VQ2_S2_NONE || pool1, "%s: NULL stage-2 plane", fn);
    CHECK(dt_ok(gu_dt) && dt_ok(s_dt) && dt_ok(out_dt), "%s: bad dtype code", fn);
    CHECK(ids_dt == VQ2_ID_I32 || ids_dt == VQ2_ID_I64, "%s: bad ids dtype", fn);
    CHECK(gu_stride >= 2 * ng * 8, "%s: gu_stride < 2 * n", fn);
    CHECK(out_stride >= out_rows, "%s: out_stride < out_rows", fn);
    CHECK(tokens <= 65535 && P <= 4096, "%s: too many tokens/pairs", fn);
    CHECK(hb >= 2 && hb <= 8192 && (hb & (hb - 1)) == 0 && (ng * 8) % hb == 0, "%s: bad hb", fn);
    if (int rr = check_rot_tables(perm, sign)) return rr;
    int r = check_codebooks(s2, cb, cb1, cb_dt);
    if (r) return r;
    GemvCall c = base_call(gu, gu_dt, s2, cb, cb1, cb_dt, s_dt, out_dt, ng, 1, rs, stream);
    c.x_bstride = gu_stride;
    c.x_pstride = gu_stride;
    c.ids = ids;
    c.ids_i64 = ids_dt == VQ2_ID_I64;
    c.n_experts = n_experts;
    c.pair_w = w;
    c.y_acc = accumulate ? 1 : 0;
    c.P = (int)P;
    c.n_out_groups = tokens;
    c.y_ostride = out_stride;
    c.nseg = 1;
    c.seg[0] = GemvSegCall{pool, pool1, pool_scale, out, out_rows, 0};
    c.xm = 2;
    c.perm = perm;
    c.sign = sign;
    c.hb = hb;
    c.xscale = rht_scale;
    return gemv_launch(c);
}

int vq2_moe_down_swiglu_combine(const void* gu, int gu_dt, int64_t gu_stride, const int32_t* perm,
                                const int8_t* sign, int64_t hb, float rht_scale, const void* ids, int ids_dt,
                                const float* w, int64_t tokens, int64_t P, const int16_t* pool, int64_t n_experts,
                                const void* cb, int cb_dt, const void* pool_scale, int s_dt, void* out, int out_dt,
                                int64_t out_stride, int64_t out_rows, int64_t ng, float rs, void* stream)
{
    return moe_down_swiglu_combine("vq2_moe_down_swiglu_combine", gu, gu_dt, gu_stride, perm, sign, hb, rht_scale,
                                   ids, ids_dt, w, tokens, P, pool, nullptr, VQ2_S2_NONE, n_experts, cb, nullptr,
                                   cb_dt, pool_scale, s_dt, out, out_dt, out_stride, out_rows, ng, rs, 0, stream);
}

int vq2_moe_down_swiglu_combine_16_8(const void* gu, int gu_dt, int64_t gu_stride, const int32_t* perm,
                                     const int8_t* sign, int64_t hb, float rht_scale, const void* ids, int ids_dt,
                                     const float* w, int64_t tokens, int64_t P, const int16_t* pool,
                                     const uint8_t* pool1, int64_t n_experts, const void* cb, const void* cb1,
                                     int cb_dt, const void* pool_scale, int s_dt, void* out, int out_dt,
                                     int64_t out_stride, int64_t out_rows, int64_t ng, float rs, int accumulate,
                                     void* stream)
{
    return moe_down_swiglu_combine("vq2_moe_down_swiglu_combine_16_8", gu, gu_dt, gu_stride, perm, sign, hb,
                                   rht_scale, ids, ids_dt, w, tokens, P, pool, pool1, VQ2_S2_U8, n_experts, cb, cb1,
                                   cb_dt, pool_scale, s_dt, out, out_dt, out_stride, out_rows, ng, rs, accumulate,
                                   stream);
}

int vq2_rht(const void* x, int x_dt, int64_t x_stride, void* y, int y_dt, int64_t y_stride, const int32_t* perm,
            const int8_t* sign, int64_t n, int64_t hb, int64_t batch, float scale, int inverse, void* stream)
{
    clear_error();
    CHECK(n > 0 && batch >= 0 && hb > 0, "vq2_rht: bad sizes");
    if (batch == 0) return VQ2_OK;
    CHECK(x && y, "vq2_rht: NULL pointer argument");
    CHECK(x != y, "vq2_rht: x and y must not overlap");
    CHECK(dt_ok(x_dt) && dt_ok(y_dt), "vq2_rht: bad dtype code");
    CHECK(x_stride >= n && y_stride >= n, "vq2_rht: strides too small");
    return rht_launch(x, x_dt, x_stride, y, y_dt, y_stride, perm, sign, n, hb, batch, scale, inverse, 0, 0, stream);
}

int vq2_swiglu_rht(const void* gu, int gu_dt, int64_t gu_stride, int64_t inter, void* y, int y_dt, int64_t y_stride,
                   const int32_t* perm, const int8_t* sign, int64_t hb, int64_t batch, float scale, void* stream)
{
    clear_error();
    CHECK(inter > 0 && batch >= 0 && hb > 0, "vq2_swiglu_rht: bad sizes");
    if (batch == 0) return VQ2_OK;
    CHECK(gu && y, "vq2_swiglu_rht: NULL pointer argument");
    CHECK(dt_ok(gu_dt) && dt_ok(y_dt), "vq2_swiglu_rht: bad dtype code");
    CHECK(gu_stride >= 2 * inter && y_stride >= inter, "vq2_swiglu_rht: strides too small");
    return rht_launch(gu, gu_dt, gu_stride, y, y_dt, y_stride, perm, sign, inter, hb, batch, scale, 0, 1, inter,
                      stream);
}

int vq2_router_topk(const void* logits, int l_dt, int64_t tokens, int64_t n_experts, int k, const void* h, int h_dt,
                    int64_t hidden, const void* gate, int g_dt, int64_t shared_id, int32_t* ids, float* w,
                    void* stream)
{
    clear_error();
    CHECK(tokens >= 0, "vq2_router_topk: bad token count");
    if (tokens == 0) return VQ2_OK;
    CHECK(logits && ids && w, "vq2_router_topk: NULL pointer argument");
    CHECK(dt_ok(l_dt), "vq2_router_topk: bad logits dtype");
    if (shared_id >= 0) {
        CHECK(h && gate && hidden > 0, "vq2_router_topk: shared gate needs h, gate and hidden");
        CHECK(dt_ok(h_dt) && dt_ok(g_dt), "vq2_router_topk: bad h/gate dtype");
    }
    return router_launch(logits, l_dt, tokens, n_experts, k, h, h_dt, hidden, gate, g_dt, shared_id, ids, w, stream);
}

int vq2_argmax_rows(const void* v, int v_dt, int64_t rows, int64_t cols, int64_t* out_idx, float* out_val,
                    void* stream)
{
    clear_error();
    CHECK(rows >= 0 && cols > 0, "vq2_argmax_rows: bad sizes");
    if (rows == 0) return VQ2_OK;
    CHECK(v && out_idx, "vq2_argmax_rows: NULL pointer argument");
    CHECK(dt_ok(v_dt), "vq2_argmax_rows: bad dtype");
    CHECK((uintptr_t)out_idx % 8 == 0, "vq2_argmax_rows: out_idx must be 8-byte aligned");
    return argmax_launch(v, v_dt, rows, cols, out_idx, out_val, stream);
}

int vq2_gemv_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride, const int16_t* idx0, const void* idx1,
                    int s2_kind, const void* cb0, const void* cb1, int cb_dt, const void* scale, int s_dt,
                    int64_t out_rows, int64_t n, float rs, float* logits_ws, int64_t* out_idx, float* out_val,
                    void* stream)
{
    clear_error();
    CHECK(out_rows > 0, "vq2_gemv_argmax: out_rows must be > 0");
    CHECK(logits_ws && out_idx, "vq2_gemv_argmax: NULL workspace/output");
    CHECK((uintptr_t)logits_ws % 8 == 0 && (uintptr_t)out_idx % 8 == 0,
          "vq2_gemv_argmax: logits_ws and out_idx must be 8-byte aligned");
    if (batch == 1 && n > 0 && n % 8 == 0 && n <= 2048 && out_rows >= 8) {
        // fused top-1: the GEMV keeps the best key per workgroup (in the
        // logits workspace, 8 bytes per workgroup and column; a workgroup
        // covers at least 8 rows, so the keys fit) and one small launch
        // picks the winner
        CHECK(dt_ok(x_dt) && dt_ok(s_dt) && x && idx0 && scale, "vq2_gemv_argmax: bad arguments");
        CHECK(x_stride >= n, "vq2_gemv_argmax: x_stride < n");
        int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
        if (r) return r;
        CHECK((s2_kind == VQ2_S2_NONE) == (idx1 == nullptr), "vq2_gemv_argmax: idx1 must be given iff s2_kind != NONE");
        GemvCall c = base_call(x, x_dt, s2_kind, cb0, cb1, cb_dt, s_dt, VQ2_DT_F32, n / 8, batch, rs, stream);
        c.x_bstride = x_stride;
        c.nseg = 1;
        c.seg[0] = GemvSegCall{idx0, idx1, scale, logits_ws, out_rows, out_rows};
        unsigned grid_x = 0;
        c.ep = 1;
        c.cand = (uint64_t*)logits_ws;
        c.grid_x_out = &grid_x;
        r = gemv_launch(c);
        if (r == VQ2_OK) return argmax_final_launch((const uint64_t*)logits_ws, grid_x, batch, out_idx, out_val, stream);
        if (r != VQ2_ERR_UNSUPPORTED) return r;
        clear_error();  // shape outside the fused path: logits, then top-1
    }
    int r = vq2_gemv(x, x_dt, batch, x_stride, idx0, idx1, s2_kind, cb0, cb1, cb_dt, scale, s_dt, logits_ws,
                     VQ2_DT_F32, out_rows, out_rows, n, rs, stream);
    if (r) return r;
    return vq2_argmax_rows(logits_ws, VQ2_DT_F32, batch, out_rows, out_idx, out_val, stream);
}

// ------------------------------------------------------ code-sorted layout
int64_t vq2_sorted_rows_per_chunk(int64_t out_rows, int64_t ng, int64_t chunk_align)
{
    return sorted_rows_per_chunk(out_rows, ng, chunk_align);
}

int vq2_sorted_pack(const int16_t* idx0, const int16_t* idx1, int64_t out_rows, int64_t ng, int64_t rows_per_chunk,
                    uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk, int64_t* stage1_iters,
                    int64_t* n_iters, int n_threads)
{
    clear_error();
    CHECK(idx0 && entries && iters_per_chunk && stage1_iters && n_iters, "vq2_sorted_pack: NULL pointer argument");
    CHECK(out_rows >= 1 && ng >= 1, "vq2_sorted_pack: bad sizes out_rows=%lld ng=%lld", (long long)out_rows,
          (long long)ng);
    return sorted_pack(idx0, idx1, out_rows, ng, rows_per_chunk, entries, cap_iters, iters_per_chunk, stage1_iters,
                       n_iters, n_threads);
}

static int sorted_call(SortedCall& c, const char* who, const void* x, int x_dt, const int32_t* perm,
                       const int8_t* sign, int64_t hb, float rht_scale, int n_mat, const vq2_sorted_mat* mats,
                       const void* cb0, const void* cb1, int cb_dt, int s_dt, int y_dt, int64_t n, float rs,
                       int slices, void* stream)
{
    CHECK(n > 0 && n % 8 == 0, "%s: n=%lld must be a positive multiple of 8", who, (long long)n);
    CHECK(n_mat >= 1 && n_mat <= 4 && mats, "%s: 1..4 matrices", who);
    CHECK(x && cb0, "%s: NULL pointer argument", who);
    CHECK(dt_ok(x_dt) && dt_ok(s_dt) && dt_ok(y_dt), "%s: bad dtype code", who);
    CHECK(cb_dt == VQ2_DT_F16 || cb_dt == VQ2_DT_BF16, "%s: fp16 / bf16 codebooks only", who);
    CHECK(hb >= 0, "%s: bad hb", who);
    c = SortedCall{};
    c.x = x;
    c.x_dt = x_dt;
    c.xm = hb > 0 ? 1 : 0;
    c.perm = perm;
    c.sign = sign;
    c.hb = hb;
    c.xscale = rht_scale;
    c.cb0 = cb0;
    c.cb1 = cb1;
    c.cb_dt = cb_dt;
    c.s_dt = s_dt;
    c.y_dt = y_dt;
    c.ng = n / 8;
    c.rs = rs;
    c.slices = slices;
    c.nseg = n_mat;
    c.stream = stream;
    for (int i = 0; i < n_mat; i++) {
        const vq2_sorted_mat& m = mats[i];
        CHECK(m.entries && m.scale, "%s: matrix %d has a NULL pointer", who, i);
        CHECK(m.out_rows >= 1 && m.n_iters >= 1, "%s: matrix %d: bad sizes", who, i);
        CHECK(m.has_stage2 >= 0 && m.has_stage2 <= 2, "%s: matrix %d: has_stage2 must be 0, 1 or 2", who, i);
        CHECK(!m.has_stage2 || cb1, "%s: matrix %d has stage-2 entries but no cb1", who, i);
        CHECK(m.has_stage2 == mats[0].has_stage2, "%s: the matrices of a launch share one cfg", who);
        c.seg[i] = SortedSegCall{m.entries, m.iters_per_chunk, m.stage1_iters, m.n_iters, m.rows_per_chunk,
                                 m.has_stage2 ? 1 : 0, m.scale, m.y, m.out_rows};
    }
    if (!mats[0].has_stage2) c.cb1 = nullptr;
    c.cb1_rows = mats[0].has_stage2 == 2 ? 256 : 65536;
    return VQ2_OK;
}

size_t vq2_sorted_gemv_workspace(const vq2_sorted_mat* mats, int n_mat, int slices)
{
    if (!mats || n_mat < 1 || n_mat > 4 || slices <= 1) return 0;
    SortedCall c{};
    c.slices = slices;
    c.nseg = n_mat;
    for (int i = 0; i < n_mat; i++) c.seg[i].out_rows = mats[i].out_rows;
    return sorted_workspace_bytes(c);
}

int vq2_sorted_gemv(const void* x, int x_dt, const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                    int n_mat, const vq2_sorted_mat* mats, const void* cb0, const void* cb1, int cb_dt, int s_dt,
                    int y_dt, int64_t n, float rs, int slices, void* workspace, size_t ws_bytes, void* stream)
{
    clear_error();
    SortedCall c;
    int r = sorted_call(c, "vq2_sorted_gemv", x, x_dt, perm, sign, hb, rht_scale, n_mat, mats, cb0, cb1, cb_dt, s_dt,
                        y_dt, n, rs, slices, stream);
    if (r) return r;
    for (int i = 0; i < n_mat; i++) CHECK(mats[i].y, "vq2_sorted_gemv: matrix %d has no output", i);
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    return sorted_launch(c, nullptr, nullptr);
}

size_t vq2_sorted_gemv_argmax_workspace(const vq2_sorted_mat* mat)
{
    if (!mat) return 0;
    return sorted_top1_workspace_bytes(mat->out_rows, mat->rows_per_chunk);
}

int vq2_sorted_gemv_argmax(const void* x, int x_dt, const int32_t* perm, const int8_t* sign, int64_t hb,
                           float rht_scale, const vq2_sorted_mat* mat, const void* cb0, const void* cb1, int cb_dt,
                           int s_dt, int64_t n, float rs, void* workspace, size_t ws_bytes, int64_t* out_idx,
                           float* out_val, void* stream)
{
    clear_error();
    SortedCall c;
    int r = sorted_call(c, "vq2_sorted_gemv_argmax", x, x_dt, perm, sign, hb, rht_scale, 1, mat, cb0, cb1, cb_dt, s_dt,
                        VQ2_DT_F32, n, rs, 1, stream);
    if (r) return r;
    CHECK(out_idx && (uintptr_t)out_idx % 8 == 0, "vq2_sorted_gemv_argmax: out_idx must be 8-byte aligned");
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    return sorted_launch(c, out_idx, out_val);
}

size_t vq2_sorted_gemm_batch_workspace(const vq2_sorted_mat* mats, int n_mat, int64_t batch, int slices)
{
    if (!mats || n_mat < 1 || n_mat > 4 || slices <= 1 || batch < 1 || batch > 4) return 0;
    SortedCall c{};
    c.slices = slices;
    c.nseg = n_mat;
    c.batch = batch;
    for (int i = 0; i < n_mat; i++) c.seg[i].out_rows = mats[i].out_rows;
    return sorted_batch_workspace_bytes(c);
}

int vq2_sorted_gemm_batch(const void* x, int x_dt, int64_t batch, int64_t x_stride, int n_mat,
                          const vq2_sorted_mat* mats, const void* cb0, const void* cb1, int cb_dt, int s_dt, int y_dt,
                          int64_t n, float rs, int slices, void* workspace, size_t ws_bytes, void* stream)
{
    clear_error();
    SortedCall c;
    int r = sorted_call(c, "vq2_sorted_gemm_batch", x, x_dt, nullptr, nullptr, 0, 1.0f, n_mat, mats, cb0, cb1, cb_dt,
                        s_dt, y_dt, n, rs, slices, stream);
    if (r) return r;
    for (int i = 0; i < n_mat; i++) CHECK(mats[i].y, "vq2_sorted_gemm_batch: matrix %d has no output", i);
    c.batch = batch;
    c.x_stride = x_stride;
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    return sorted_batch_launch(c, nullptr, nullptr);
}

size_t vq2_sorted_gemm_batch_argmax_workspace(const vq2_sorted_mat* mat, int64_t batch)
{
    if (!mat) return 0;
    return sorted_batch_top1_workspace_bytes(mat->out_rows, mat->rows_per_chunk, batch);
}

int vq2_sorted_gemm_batch_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                                 const vq2_sorted_mat* mat, const void* cb0, const void* cb1, int cb_dt, int s_dt,
                                 int64_t n, float rs, void* workspace, size_t ws_bytes, int64_t* out_idx,
                                 float* out_val, void* stream)
{
    clear_error();
    SortedCall c;
    int r = sorted_call(c, "vq2_sorted_gemm_batch_argmax", x, x_dt, nullptr, nullptr, 0, 1.0f, 1, mat, cb0, cb1,
                        cb_dt, s_dt, VQ2_DT_F32, n, rs, 1, stream);
    if (r) return r;
    CHECK(out_idx && (uintptr_t)out_idx % 8 == 0, "vq2_sorted_gemm_batch_argmax: out_idx must be 8-byte aligned");
    c.batch = batch;
    c.x_stride = x_stride;
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    return sorted_batch_launch(c, out_idx, out_val);
}

int vq2_sorted_pack_pool(const int16_t* idx, const int16_t* idx1, int64_t n_experts, int64_t rows, int64_t ng,
                         int64_t rows_per_chunk, uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk,
                         int64_t* stage1_iters, int64_t* n_iters, int n_threads)
{
    clear_error();
    CHECK(idx && entries && iters_per_chunk && stage1_iters && n_iters, "vq2_sorted_pack_pool: NULL pointer argument");
    CHECK(n_experts >= 1 && rows >= 1 && ng >= 1, "vq2_sorted_pack_pool: bad sizes n_experts=%lld rows=%lld ng=%lld",
          (long long)n_experts, (long long)rows, (long long)ng);
    return sorted_pack_pool(idx, idx1, n_experts, rows, ng, rows_per_chunk, entries, cap_iters, iters_per_chunk,
                            stage1_iters, n_iters, n_threads);
}

size_t vq2_sorted_moe_workspace(int64_t tokens, int pairs_per_token, int64_t hidden, int64_t inter, int slices_gu,
                                int slices_dn)
{
    if (tokens < 1 || pairs_per_token < 1 || hidden < 1 || inter < 1 || slices_gu < 1 || slices_dn < 1) return 0;
    return sorted_moe_workspace_bytes(tokens * pairs_per_token, hidden, inter, slices_gu, slices_dn);
}

int vq2_sorted_moe_status(void* workspace, int clear, void* stream)
{
    clear_error();
    CHECK(workspace, "vq2_sorted_moe_status: NULL workspace");
    hipStream_t st = (hipStream_t)stream;
    uint32_t* word = (uint32_t*)((char*)workspace + VQ2_SORTED_WS_STATUS);
    uint32_t v = 0;
    hipError_t err = hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, st);
    if (err == hipSuccess) err = hipStreamSynchronize(st);
    if (err == hipSuccess && clear) {
        static const uint32_t zero = 0;
        err = hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, st);
        if (err == hipSuccess) err = hipStreamSynchronize(st);
    }
    if (err != hipSuccess) return set_hip_error(err, "vq2_sorted_moe_status");
    return (int)(v & 0x7FFFFFFFu);
}

int vq2_sorted_moe_set_wait(int64_t max_polls, int32_t extra_arrivals)
{
    clear_error();
    return sorted_moe_set_wait(max_polls, extra_arrivals);
}

int vq2_sorted_moe(const void* h, int h_dt, int64_t tokens, int pairs_per_token, const void* ids, int ids_i64,
                   const float* w, const void* logits, int l_dt, int64_t n_routed, int top_k, int64_t shared_id,
                   const void* shared_gate, int g_dt, int32_t* ids_out, float* w_out, int64_t n_experts,
                   int64_t hidden, int64_t inter, const vq2_sorted_pool* gate_up, const vq2_sorted_pool* down,
                   const void* cb, int cb_dt, const vq2_rot_tables* rot_h, const vq2_rot_tables* rot_i, void* out,
                   int out_dt, int slices_gu, int slices_dn, void* workspace, size_t ws_bytes, void* stream)
{
    clear_error();
    CHECK(gate_up && down && rot_h && rot_i, "vq2_sorted_moe: NULL pool or rotation");
    SortedMoeCall c{};
    c.h = h;
    c.h_dt = h_dt;
    c.tokens = tokens;
    c.P = pairs_per_token;
    c.ids = ids;
    c.ids_i64 = ids_i64;
    c.w = w;
    c.logits = logits;
    c.l_dt = l_dt;
    c.n_routed = n_routed;
    c.top_k = top_k;
    c.shared_id = shared_id;
    c.shared_gate = shared_gate;
    c.g_dt = g_dt;
    c.ids_out = ids_out;
    c.w_out = w_out;
    c.n_experts = n_experts;
    c.hidden = hidden;
    c.inter = inter;
    c.gate_up = SortedPoolCall{gate_up->entries, gate_up->iters_per_chunk, gate_up->stage1_iters, gate_up->has_stage2,
                               gate_up->cb1, gate_up->n_iters, gate_up->rows_per_chunk, gate_up->rows, gate_up->ng,
                               gate_up->scale, gate_up->scale_dt};
    c.down = SortedPoolCall{down->entries, down->iters_per_chunk, down->stage1_iters, down->has_stage2, down->cb1,
                            down->n_iters, down->rows_per_chunk, down->rows, down->ng, down->scale, down->scale_dt};
    c.cb = cb;
    c.cb_dt = cb_dt;
    c.rot_h = SortedRot{rot_h->perm, rot_h->sign, rot_h->hb, rot_h->scale};
    c.rot_i = SortedRot{rot_i->perm, rot_i->sign, rot_i->hb, rot_i->scale};
    c.out = out;
    c.out_dt = out_dt;
    c.slices_gu = slices_gu;
    c.slices_dn = slices_dn;
    c.workspace = workspace;
    c.ws_bytes = ws_bytes;
    c.stream = stream;
    return sorted_moe_launch(c);
}

size_t vq2_pager_lds_bytes(int64_t n_experts, int64_t capacity, int64_t n_pairs)
{
    return pager_lds_bytes(n_experts, capacity, n_pairs);
}

int vq2_pager_step(const void* ids, int ids_i64, int64_t n_pairs, int64_t n_experts, int64_t capacity,
                   int32_t* slot_of, int32_t* expert_of, int32_t* stamp, int32_t* state, int32_t* copy_list,
                   int32_t* pair_slot, void* stream)
{
    clear_error();
    CHECK(n_pairs >= 1 && n_pairs <= 4096 && n_experts >= 1 && n_experts <= 65536 && capacity >= 1 &&
              capacity <= 4096, "vq2_pager_step: bad sizes (pairs %lld, experts %lld, slots %lld)", (long long)n_pairs,
          (long long)n_experts, (long long)capacity);
    CHECK(ids && slot_of && expert_of && stamp && state && copy_list && pair_slot, "vq2_pager_step: NULL pointer");
    return pager_step_launch(ids, ids_i64, n_pairs, n_experts, capacity, slot_of, expert_of, stamp, state, copy_list,
                             pair_slot, stream);
}

int vq2_pager_copy(const void* mirror, int64_t record_bytes, const int64_t* seg_bytes, const int32_t* copy_list,
                   const int32_t* state, int64_t max_copies, void* const* dst, const int64_t* dst_stride, int scale_dt,
                   void* stream)
{
    clear_error();
    CHECK(mirror && seg_bytes && copy_list && state && dst && dst_stride, "vq2_pager_copy: NULL pointer");
    CHECK(dt_ok(scale_dt), "vq2_pager_copy: bad scale dtype");
    return pager_copy_launch(mirror, record_bytes, seg_bytes, copy_list, state, max_copies, dst, dst_stride, scale_dt,
                             stream);
}

int vq2_dequant_rows(const int16_t* idx0, const void* idx1, int s2_kind, const void* cb0, const void* cb1, int cb_dt,
                     const void* scale, int s_dt, int64_t r0, int64_t r1, int64_t n, float* out, void* stream)
{
    clear_error();
    CHECK(r0 >= 0 && r1 >= r0 && n > 0 && n % 8 == 0, "vq2_dequant_rows: bad row range or n");
    if (r1 == r0) return VQ2_OK;
    CHECK(idx0 && scale && out, "vq2_dequant_rows: NULL pointer argument");
    CHECK(dt_ok(s_dt), "vq2_dequant_rows: bad scale dtype");
    int r = check_codebooks(s2_kind, cb0, cb1, cb_dt);
    if (r) return r;
    CHECK((s2_kind == VQ2_S2_NONE) == (idx1 == nullptr), "vq2_dequant_rows: idx1 must be given iff s2_kind != NONE");
    return dequant_launch(idx0, idx1, s2_kind, cb0, cb1, cb_dt, scale, s_dt, r0, r1, n, out, stream);
}

int vq2_decode_idx(const void* in, int is_u8, int64_t count, int32_t* out, void* stream)
{
    clear_error();
    CHECK(count >= 0, "vq2_decode_idx: bad count");
    if (count == 0) return VQ2_OK;
    CHECK(in && out, "vq2_decode_idx: NULL pointer argument");
    return decode_launch(in, is_u8, count, out, stream);
}

int vq2_unpack_fixed(const uint8_t* buf, int64_t nbytes, int bits, int64_t n, int16_t* out, void* stream)
{
    clear_error();
    CHECK(n >= 0 && nbytes >= 0, "vq2_unpack_fixed: bad sizes");
    if (n == 0) return VQ2_OK;
    CHECK(buf && out, "vq2_unpack_fixed: NULL pointer argument");
    return unpack_fixed_launch(buf, nbytes, bits, n, out, stream);
}

}  // extern "C"
