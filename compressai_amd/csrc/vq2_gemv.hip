// vq2_gemv.hip -- launch planning and dispatch of the VQ GEMV kernels
// (kernel bodies and design notes: vq2_gemv_kernel.hpp).
#include <stdlib.h>

#include <map>
#include <mutex>
#include <tuple>

#include "vq2_gemv_kernel.hpp"

namespace vq2 {

// LDS the planner allows per workgroup (two workgroups per CU stay resident)
constexpr int64_t GEMV_LDS_BUDGET = 64 * 1024;

// Tuning override read once from the environment (VQ2_GEMV_OCC_SCALE:
// multiplier on the resident-workgroup grid).
static double env_double(const char* name, double dflt)
{
    const char* v = getenv(name);
    return v ? atof(v) : dflt;
}

int resident_blocks_per_cu(const void* fn, int threads, size_t shm)
{
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t, int>, int> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    const auto key = std::make_tuple(fn, threads, shm, dev);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, threads, shm) != hipSuccess || nb < 1) nb = 1;
    cache[key] = nb;
    return nb;
}

static GemvPlan plan_gemv(const GemvCall& c, int num_cu)
{
    GemvPlan p;
    const int batch = (int)c.batch;
    const int P = c.P > 0 ? c.P : 1;
    p.xm = c.xm;
    p.bt = batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8;
    p.gpl = 8 / p.bt;  // activation slice per lane stays at 64 fp32 values
    const int64_t need = (c.ng + p.gpl - 1) / p.gpl;
    int lpr = 1;
    while (lpr < need && lpr < 32) lpr <<= 1;
    p.lpr = lpr;
    const int64_t kc = (int64_t)lpr * p.gpl;
    const int64_t nch = (c.ng + kc - 1) / kc;
    const int64_t items = (int64_t)P * nch;
    if (items <= 4) {
        p.wi = (int)items;
        p.wr = 4 / p.wi;
    } else {
        // more items than 4 waves: up to the kernel's wave limit, balanced so
        // that every wave runs the same number of item rounds (a wave's
        // items run one after the other, each a full index + gather latency)
        const int64_t wi_max = gemv_max_threads(c.s2, c.cb_dt, c.xm) / 64;
        const int64_t rounds = (items + wi_max - 1) / wi_max;
        p.wi = wi_max <= 4 ? 4 : (int)((items + rounds - 1) / rounds);
        p.wr = 1;
    }
    // RHT prologue wider than one pass of the 4-wave workgroup (8 values per
    // thread): XM 4, with enough waves along rows that one pass covers the
    // activation block (its loads are issued before the index words and its
    // arithmetic overlaps the first gathers; later passes would wait behind
    // them)
    if (p.xm == 1) {
        const int64_t x_vals = (int64_t)p.bt * c.ng * 8;
        const int64_t waves = (x_vals / 8 + 63) / 64;
        if (waves > (int64_t)p.wi * p.wr) {
            const int64_t wr = (waves + p.wi - 1) / p.wi;
            if (64 * p.wi * wr <= gemv_max_threads(c.s2, c.cb_dt, 4)) {
                p.xm = 4;
                p.wr = (int)wr;
            }
        }
    }
    p.threads = 64 * p.wi * p.wr;
    const int rpw = 64 / lpr;
    const int64_t ztiles = (batch + p.bt - 1) / p.bt;
    int64_t max_rows = 0;
    for (int s = 0; s < c.nseg; s++) max_rows = c.seg[s].out_rows > max_rows ? c.seg[s].out_rows : max_rows;
    p.it = p.bt == 8 ? gemv_it<8>() : gemv_it<1>();
    static const double occ_env = env_double("VQ2_GEMV_OCC_SCALE", 1.0);
    p.occ_scale = occ_env > 0 ? occ_env : 1.0;
    p.num_cu = num_cu;
    p.ep = c.ep;
    p.grid_x_out = c.grid_x_out;
    p.rows_per_block = (int64_t)p.it * rpw * p.wr;
    p.n_rowblocks = 0;
    for (int s = 0; s < c.nseg; s++) p.n_rowblocks += (c.seg[s].out_rows + p.rows_per_block - 1) / p.rows_per_block;
    (void)ztiles;
    (void)max_rows;
    return p;
}

hipError_t gemv_generic_dispatch(int cb_dt, int s2, int si, const GemvArgs& a, dim3 grid, hipStream_t st)
{
    switch (cb_dt) {
    case VQ2_DT_F16: return launch_generic<VQ2_DT_F16>(s2, si, a, grid, st);
    case VQ2_DT_BF16: return launch_generic<VQ2_DT_BF16>(s2, si, a, grid, st);
    default: return launch_generic<VQ2_DT_F32>(s2, si, a, grid, st);
    }
}

int gemv_launch(const GemvCall& c)
{
    if (c.batch == 0 || c.n_out_groups == 0 || c.nseg == 0) return VQ2_OK;
    if (c.nseg < 0 || c.nseg > VQ2_MAX_SEG) return set_error(VQ2_ERR_ARG, "vq2 gemv: 1..%d segments", VQ2_MAX_SEG);
    if (c.n_out_groups > 65535) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: too many output groups");
    if (c.batch > 0x7FFFFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: batch too large");
    GemvArgs a{};
    a.x = c.x;
    a.x_dt = c.x_dt;
    a.x_bstride = c.x_bstride;
    a.x_pstride = c.x_pstride;
    a.x_pdiv = c.x_pdiv > 0 ? c.x_pdiv : 1;
    a.cb0 = c.cb0;
    a.cb1 = c.cb1;
    a.s_dt = c.s_dt;
    a.ids = c.ids;
    a.ids_i64 = c.ids_i64;
    a.n_experts = c.n_experts;
    a.pair_w = c.pair_w;
    a.y_acc = c.y_acc;
    a.P = c.P > 0 ? c.P : 1;
    a.y_dt = c.y_dt;
    a.y_ostride = c.y_ostride;
    a.ng = c.ng;
    a.batch = (int)c.batch;
    a.rs = c.rs;
    a.nseg = c.nseg;
    a.e_istride = c.seg[0].out_rows * c.ng;  // grouped launches have one segment
    a.e_sstride = c.seg[0].out_rows;
    a.perm = c.perm;
    a.sign = c.sign;
    a.xscale = c.xscale;
    a.r_logits = c.r_logits;
    a.r_ldt = c.r_ldt;
    a.r_ne = c.r_ne;
    a.r_k = c.r_k;
    a.r_pairs = c.r_pairs > 0 ? c.r_pairs : 1;
    a.r_shared = c.r_shared;
    a.r_gate = c.r_gate;
    a.r_gdt = c.r_gdt;
    a.r_ids = c.r_ids;
    a.r_w = c.r_w;
    a.cand = c.cand;
    int L = 0;
    if (c.xm != 0) {
        while ((1LL << L) < c.hb) L++;
        if (L < 1 || L > 13 || (1LL << L) != c.hb || (c.ng * 8) % c.hb)
            return set_error(VQ2_ERR_ARG, "vq2 gemv: hb=%lld must be a power of two in [2, 8192] dividing n=%lld",
                             (long long)c.hb, (long long)(c.ng * 8));
    }
    a.hb_log2 = L;
    hipStream_t st = (hipStream_t)c.stream;
    const int num_cu = device_cu_count();
    const GemvPlan p = plan_gemv(c, num_cu);
    if (p.n_rowblocks == 0) return VQ2_OK;  // every segment has zero rows

    // the vector kernel needs GPL-wide, aligned index words and 16-byte
    // aligned activation rows
    uintptr_t ia = 0, i8 = 0;
    for (int s = 0; s < c.nseg; s++) {
        ia |= (uintptr_t)c.seg[s].idx0;
        if (c.s2 == VQ2_S2_U16) ia |= (uintptr_t)c.seg[s].idx1;
        if (c.s2 == VQ2_S2_U8) i8 |= (uintptr_t)c.seg[s].idx1;
    }
    const int64_t esz_x = dt_size(c.x_dt);
    const bool x_vec = c.xm != 0 || (((uintptr_t)c.x % 16 == 0) && ((c.x_bstride * esz_x) % 16 == 0) &&
                                     ((c.x_pstride * esz_x) % 16 == 0));
    const bool vec_ok = x_vec && (c.ng % p.gpl == 0) && (ia % (2 * p.gpl) == 0) && (i8 % p.gpl == 0);
    hipError_t err;
    if (c.ep == 1) {
        // the fused top-1 runs in the one-item-per-wave path of the vector kernel
        const int64_t nch = (c.ng + (int64_t)p.lpr * p.gpl - 1) / ((int64_t)p.lpr * p.gpl);
        if (!vec_ok || c.xm != 0 || c.nseg != 1 || (c.P > 1) || nch != 1 || p.bt != 1 || p.it != 1 || !c.cand)
            return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: the fused top-1 does not apply to this shape");
    }
    if (!vec_ok) {
        if (c.xm != 0)
            return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: the fused rotation needs n %% 64 == 0 and aligned planes");
        for (int s = 0; s < c.nseg; s++) {
            a.seg[s] = GemvSeg{c.seg[s].idx0, c.seg[s].idx1, c.seg[s].scale, c.seg[s].y, c.seg[s].out_rows,
                               c.seg[s].y_bstride, 0};
            const int64_t work = c.batch * c.seg[s].out_rows;
            int64_t blocks = (work + 255) / 256;
            if (blocks > 4LL * num_cu) blocks = 4LL * num_cu;
            if (blocks == 0) continue;
            err = gemv_generic_dispatch(c.cb_dt, c.s2, s, a, dim3((unsigned)blocks, (unsigned)c.n_out_groups), st);
            if (err != hipSuccess) return set_hip_error(err, "vq2 gemv (generic) launch");
        }
        return VQ2_OK;
    }

    int64_t rb = 0;
    for (int s = 0; s < c.nseg; s++) {
        a.seg[s] = GemvSeg{c.seg[s].idx0, c.seg[s].idx1, c.seg[s].scale, c.seg[s].y, c.seg[s].out_rows,
                           c.seg[s].y_bstride, rb};
        rb += (c.seg[s].out_rows + p.rows_per_block - 1) / p.rows_per_block;
    }
    // unused segment slots start past every row block: seg_of() needs no nseg
    for (int s = c.nseg; s < VQ2_MAX_SEG; s++) a.seg[s].rb_start = INT64_MAX;
    a.lpr = p.lpr;
    a.wi = p.wi;
    a.nch = (int)((c.ng + (int64_t)p.lpr * p.gpl - 1) / ((int64_t)p.lpr * p.gpl));
    a.n_rowblocks = p.n_rowblocks;
    // the kernel's packed scalar arguments
    if (c.ng > 0x7FFFFFFF || p.n_rowblocks > 0x7FFFFFFF || c.seg[0].out_rows > 0x7FFFFFFF || a.nch > 0xFFFF ||
        a.P > 0xFFFF || p.lpr > 63 || p.wi > 15 || p.wr > 15)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: shape outside the kernel's argument ranges");
    if (p.threads > gemv_max_threads(c.s2, c.cb_dt, p.xm) || p.threads % 64)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: internal plan error (%d threads)", p.threads);
    if (c.xm == 2 && (c.s2 == VQ2_S2_U16 || p.bt != 1))
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: the fused SwiGLU prologue is for 2 and 3 bpw, batch 1");
    if (c.xm == 3 && (c.s2 != VQ2_S2_NONE || p.bt != 1 || !c.r_logits))
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: the fused router is for 2 bpw, batch 1");
    if (c.xm == 1 && p.bt > 2)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: the fused rotation supports batch <= 2 per launch");
    const int64_t ztiles = (c.batch + p.bt - 1) / p.bt;
    if (ztiles > 65535) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: too many batch tiles");
    // grid.x is set per kernel from its resident-workgroup count
    dim3 grid(1, (unsigned)c.n_out_groups, (unsigned)ztiles);
    const int64_t items = (int64_t)a.P * ((c.ng + (int64_t)p.lpr * p.gpl - 1) / ((int64_t)p.lpr * p.gpl));
    const int64_t x_floats = c.xm == 0 ? 0 : (c.xm == 2 ? (int64_t)a.P : p.bt) * c.ng * 8;
    const int64_t part_floats = items > 1 ? (int64_t)p.wi * p.rows_per_block * p.bt : 0;
    // the prologue stages the unpermuted activation block where the partials go later: raw
    // elements, or silu(gate) * up as fp32 for XM 2
    const int64_t stage_floats = c.xm == 0 ? 0 : c.xm == 2 ? x_floats : (x_floats * dt_size(c.x_dt) + 3) / 4;
    const size_t shm = (size_t)(x_floats + std::max(part_floats, stage_floats)) * sizeof(float);
    if ((int64_t)shm > GEMV_LDS_BUDGET)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: %zu bytes of LDS needed (> %lld)", shm,
                         (long long)GEMV_LDS_BUDGET);
    switch (c.cb_dt) {
    case VQ2_DT_F16: err = gemv_dispatch_f16(c.s2, a, p, grid, shm, st); break;
    case VQ2_DT_BF16: err = gemv_dispatch_bf16(c.s2, a, p, grid, shm, st); break;
    default: err = gemv_dispatch_f32(c.s2, a, p, grid, shm, st); break;
    }
    if (err != hipSuccess) return set_hip_error(err, "vq2 gemv launch");
    return VQ2_OK;
}

}  // namespace vq2
