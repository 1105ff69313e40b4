// vq2_gemv.hip -- launch planning and dispatch of the VQ GEMV kernel
// (kernel body and design notes: vq2_gemv_kernel.hpp).
#include "vq2_gemv_kernel.hpp"

namespace vq2 {

static GemvPlan plan_gemv(int64_t out_rows, int64_t ng, int batch, int64_t n_out_groups, int P, int num_cu)
{
    GemvPlan p;
    p.bt = batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8;
    p.gpl = 8 / p.bt;
    int64_t need = (ng + p.gpl - 1) / p.gpl;
    int lpr = 1;
    while (lpr < need && lpr < 32) lpr <<= 1;
    p.lpr = lpr;
    const int64_t kc = (int64_t)lpr * p.gpl;
    const int64_t nch = (ng + kc - 1) / kc;
    p.wk = (int)(nch < 4 ? nch : 4);  // <= 4 waves: the kernel is built for 256-thread workgroups
    p.wr = p.wk >= 4 ? 1 : 4 / p.wk;
    p.threads = 64 * p.wk * p.wr;
    const int rpw = 64 / lpr;
    const int64_t ztiles = (batch + p.bt - 1) / p.bt;
    const bool use_lds = p.wk > 1 || P > 1;
    // rows per lane: as many as keep >= 4 workgroups per CU busy
    p.it = 1;
    for (int it = 4; it >= 2; it >>= 1) {
        const int64_t rpi = (int64_t)it * rpw * p.wr;
        const int64_t blocks = (out_rows + rpi - 1) / rpi;
        if (use_lds && rpi * p.bt > p.threads) continue;
        if (blocks * n_out_groups * ztiles >= 4LL * num_cu) { p.it = it; break; }
    }
    p.rows_per_iter = (int64_t)p.it * rpw * p.wr;
    p.n_rowblocks = (out_rows + p.rows_per_iter - 1) / p.rows_per_iter;
    return p;
}

int gemv_launch(const GemvCall& c)
{
    if (c.out_rows == 0 || c.batch == 0 || c.n_out_groups == 0) return VQ2_OK;
    GemvArgs a{};
    a.x = c.x;
    a.x_dt = c.x_dt;
    a.x_bstride = c.x_bstride;
    a.x_pstride = c.x_pstride;
    a.x_pdiv = c.x_pdiv > 0 ? c.x_pdiv : 1;
    a.idx0 = c.idx0;
    a.idx1 = c.idx1;
    a.cb0 = c.cb0;
    a.cb1 = c.cb1;
    a.scale = c.scale;
    a.s_dt = c.s_dt;
    a.e_istride = c.out_rows * c.ng;
    a.e_sstride = c.out_rows;
    a.ids = c.ids;
    a.ids_i64 = c.ids_i64;
    a.n_experts = c.n_experts;
    a.pair_w = c.pair_w;
    a.P = c.P > 0 ? c.P : 1;
    a.y = c.y;
    a.y_dt = c.y_dt;
    a.y_bstride = c.y_bstride;
    a.y_ostride = c.y_ostride;
    a.out_rows = c.out_rows;
    a.ng = c.ng;
    a.batch = (int)c.batch;
    a.rs = c.rs;

    const GemvPlan p = plan_gemv(c.out_rows, c.ng, (int)c.batch, c.n_out_groups, a.P, device_cu_count());
    a.lpr = p.lpr;
    a.wk = p.wk;
    a.n_rowblocks = p.n_rowblocks;
    const bool use_lds = p.wk > 1 || a.P > 1;
    if (p.threads > 256 || p.threads % 64)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: internal plan error (%d threads)", p.threads);
    if (use_lds && p.rows_per_iter * p.bt > p.threads)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: combine/split-K tile does not fit (rows %lld, batch tile %d)",
                         (long long)p.rows_per_iter, p.bt);

    // vector loads need 16/8/4-byte aligned index words and activation rows
    const int64_t esz_x = c.x_dt == VQ2_DT_F32 ? 4 : 2;
    const uintptr_t ia = (uintptr_t)c.idx0 | (uintptr_t)(c.idx1 ? c.idx1 : c.idx0);
    const int idx_align = p.gpl * 2;
    a.vec_ok = (c.ng % p.gpl == 0) && (ia % idx_align == 0) &&
               (c.s2 != VQ2_S2_U8 || ((uintptr_t)c.idx1 % p.gpl == 0));
    a.x_vec = ((uintptr_t)c.x % 16 == 0) && ((c.x_bstride * esz_x) % 16 == 0) && ((c.x_pstride * esz_x) % 16 == 0);

    const int64_t ztiles = (c.batch + p.bt - 1) / p.bt;
    if (ztiles > 65535 || c.n_out_groups > 65535)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 gemv: too many pairs/batch tiles");
    const int64_t cap = 8LL * device_cu_count();
    const int64_t gx = p.n_rowblocks < cap ? p.n_rowblocks : cap;
    dim3 grid((unsigned)gx, (unsigned)c.n_out_groups, (unsigned)ztiles);
    const size_t shm = use_lds ? (size_t)p.wk * p.rows_per_iter * p.bt * sizeof(float) : 0;
    hipStream_t st = (hipStream_t)c.stream;
    hipError_t err;
    switch (c.cb_dt) {
    case VQ2_DT_F16: err = gemv_dispatch_f16(c.s2, a, p, grid, shm, st); break;
    case VQ2_DT_BF16: err = gemv_dispatch_bf16(c.s2, a, p, grid, shm, st); break;
    default: err = gemv_dispatch_f32(c.s2, a, p, grid, shm, st); break;
    }
    if (err != hipSuccess) return set_hip_error(err, "vq2 gemv launch");
    return VQ2_OK;
}

}  // namespace vq2
