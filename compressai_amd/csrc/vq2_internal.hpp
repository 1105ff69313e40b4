// vq2_internal.hpp -- host-side internals shared by the libvq2_amd sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq2_amd.h"

namespace vq2 {

// Record a formatted error message for vq2_last_error(); returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int set_hip_error(hipError_t err, const char* what);
void clear_error();

// Compute-unit count of the current device (cached per device).
int device_cu_count();

// One matrix of a GEMV launch (segments of one launch share the activation).
struct GemvSegCall {
    const int16_t* idx0;
    const void* idx1;
    const void* scale;
    void* y;
    int64_t out_rows;
    int64_t y_bstride;  // elements between batch columns of y
};

// One launch of the shared GEMV kernel body (dense / grouped / combine).
struct GemvCall {
    const void* x;
    int x_dt;
    int64_t x_bstride;  // elements between batch columns of one x block
    int64_t x_pstride;  // elements between x blocks
    int x_pdiv;         // pair p reads x block p / x_pdiv
    int s2;
    const void* cb0;
    const void* cb1;
    int cb_dt;
    int s_dt;
    const void* ids;  // null: expert 0 for every pair
    int ids_i64;
    int64_t n_experts;
    const float* pair_w;  // combine weights
    int y_acc;            // xm 2: out += combine
    int P;                // pairs per output group
    int64_t n_out_groups; // grid.y
    int y_dt;
    int64_t y_ostride;
    int64_t ng;
    int64_t batch;
    float rs;
    void* stream;
    int nseg;
    GemvSegCall seg[4];
    // activation prologue: 0 = x is the rotated activation; 1 = rotate x in
    // the kernel; 2 = rotate silu(gate) * up of each pair in the kernel
    int xm;
    const int32_t* perm;
    const int8_t* sign;
    int64_t hb;
    float xscale;
    // fused router of the gate_up launch (see GemvArgs); r_logits null = off
    const void* r_logits;
    int r_ldt;
    int64_t r_ne;
    int r_k;
    int r_pairs;
    int64_t r_shared;
    const void* r_gate;
    int r_gdt;
    int32_t* r_ids;
    float* r_w;
    // epilogue: 0 store y; 1 fused top-1 (pre-rotated x, one item per wave):
    // per-workgroup best keys to cand[grid.x][batch], grid.x to grid_x_out
    int ep;
    uint64_t* cand;
    unsigned* grid_x_out;
};

int gemv_launch(const GemvCall& c);

// Top-1 of each batch column over per-workgroup candidate keys.
int argmax_final_launch(const uint64_t* cand, int64_t n_cand, int64_t batch, int64_t* out_idx, float* out_val,
                        void* stream);

// Small-M batched GEMM on the matrix cores (vq2_gemm_mfma.hip).
struct GemmCall {
    const void* x;
    int x_dt;
    int64_t x_stride;  // elements between activation rows
    int64_t m;         // activation rows (1..64)
    const int16_t* idx0;
    const void* idx1;
    int s2;
    const void* cb0;
    const void* cb1;
    int cb_dt;
    const void* scale;
    int s_dt;
    void* y;
    int y_dt;
    int64_t y_stride;  // elements between output rows of y ([m][out_rows])
    int64_t out_rows;
    int64_t ng;
    float rs;
    void* workspace;
    size_t ws_bytes;
    void* stream;
};

size_t gemm_small_m_workspace_bytes(int64_t m, int64_t out_rows, int64_t ng);
int gemm_small_m_launch(const GemmCall& c);
// the same GEMM with its split-K partials in the library's device scratch
// (c.workspace / c.ws_bytes ignored); shapes needing more are rejected
constexpr size_t MM_NOALLOC_SCRATCH_BYTES = VQ2_NOALLOC_SCRATCH_BYTES;
int gemm_small_m_noalloc_launch(GemmCall c);
// the GEMM with the top-1 of every activation row instead of y (c.y unused)
size_t gemm_small_m_top1_workspace_bytes(int64_t m, int64_t out_rows, int64_t ng);
int gemm_small_m_top1_launch(const GemmCall& c, int64_t* out_idx, float* out_val);

// VQ GEMV over the code-sorted internal layout (vq2_sorted.hip).
struct SortedSegCall {
    const uint32_t* entries;   // [n_iters * 192] (768 bytes per iteration), 16-byte aligned
    int64_t iters_per_chunk;   // every chunk padded to it
    int64_t stage1_iters;      // of which stage 1 (the stage-2 iterations follow)
    int64_t n_iters;
    int64_t rows_per_chunk;
    int s2;                    // stage-2 entries present (4 bpw)
    const void* scale;
    void* y;
    int64_t out_rows;
};

struct SortedCall {
    const void* x;
    int x_dt;
    int xm;  // 0: x is rotated; 1: rotate x in the kernel (perm / sign / hb / xscale)
    const int32_t* perm;
    const int8_t* sign;
    int64_t hb;
    float xscale;
    const void* cb0;
    const void* cb1;
    int64_t cb1_rows = 65536;  // 256: the uint8 stage 2 of (16,8) (codes masked to 8 bits)
    int cb_dt;
    int s_dt;
    int y_dt;
    int64_t ng;
    float rs;
    int slices;
    int nseg;
    SortedSegCall seg[4];
    void* workspace;
    size_t ws_bytes;
    void* stream;
    int64_t batch = 1;     // activation rows (sorted_batch_launch: 1..4)
    int64_t x_stride = 0;  // sorted_batch_launch: elements between activation rows
};

int64_t sorted_rows_per_chunk(int64_t out_rows, int64_t ng, int64_t chunk_align);
// Checks shared by the sorted launches (`who` prefixes the messages): the
// matrix count, chunk heights (*rmax: the tallest), codebook dtype and
// alignment, slices, and the top-1's single matrix and slice; then, per
// matrix, its iteration count, entry alignment, stage-2 codebook and
// iterations = chunks x iterations per chunk (*ks: its chunks).
struct ChunkSplit;
int sorted_check_call(const SortedCall& c, bool top1, const char* who, int64_t* rmax);
// floats of one wave's accumulator arrays for the launch's tallest need:
// max over its matrices of sorted_parts(R) x (R + 1)
int64_t sorted_acc_arrays(const SortedCall& c);
int sorted_check_seg(const SortedCall& c, int s, const char* who, ChunkSplit* ks);
size_t sorted_batch_workspace_bytes(const SortedCall& c);
size_t sorted_batch_top1_workspace_bytes(int64_t out_rows, int64_t rows_per_chunk, int64_t batch);
int sorted_batch_launch(const SortedCall& c, int64_t* top1_idx, float* top1_val);
int sorted_pack(const int16_t* idx0, const int16_t* idx1, int64_t out_rows, int64_t ng, int64_t rows_per_chunk,
                uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk, int64_t* stage1_iters,
                int64_t* n_iters, int n_threads);
size_t sorted_workspace_bytes(const SortedCall& c);
size_t sorted_top1_workspace_bytes(int64_t out_rows, int64_t rows_per_chunk);
// top1_idx non-null: fused top-1 (one matrix, one slice) instead of y
int sorted_launch(const SortedCall& c, int64_t* top1_idx, float* top1_val);

// MoE experts over code-sorted expert pools (vq2_sorted_moe.hip).
int sorted_pack_pool(const int16_t* idx, const int16_t* idx1, int64_t n_experts, int64_t rows, int64_t ng,
                     int64_t rows_per_chunk, uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk,
                     int64_t* stage1_iters, int64_t* n_iters, int n_threads);

// The one-launch MoE's wait bound (polls) and arrival target offset.
struct MoeWait {
    int max_polls;
    int extra_arrivals;
};
MoeWait sorted_moe_wait();
int sorted_moe_set_wait(int64_t max_polls, int32_t extra_arrivals);

struct SortedPoolCall {
    const uint32_t* entries;
    int64_t iters_per_chunk;  // every chunk padded to this many iterations
    int64_t stage1_iters;     // of which stage 1 (the stage-2 ones follow)
    int s2;                   // 0 none, 1 int16 stage 2 (cb1 [65536, 8]), 2 uint8 stage 2 (cb1 [256, 8])
    const void* cb1;
    int64_t n_iters;
    int64_t rows_per_chunk;
    int64_t rows;  // rows per expert
    int64_t ng;    // groups per row
    const void* scale;
    int scale_dt;
};

struct SortedRot {
    const int32_t* perm;
    const int8_t* sign;
    int64_t hb;
    float scale;
};

struct SortedMoeCall {
    const void* h;
    int h_dt;
    int64_t tokens;
    int P;  // pairs per token
    // routing given: ids [tokens * P] (int32 / int64), w [tokens * P]
    const void* ids;
    int ids_i64;
    const float* w;
    // or the fused router (logits non-null): P = top_k + 1, slot top_k the
    // shared expert; writes ids_out / w_out
    const void* logits;
    int l_dt;
    int64_t n_routed;
    int top_k;
    int64_t shared_id;
    const void* shared_gate;
    int g_dt;
    int32_t* ids_out;
    float* w_out;
    int64_t n_experts;
    int64_t hidden;
    int64_t inter;
    SortedPoolCall gate_up;
    SortedPoolCall down;
    const void* cb;
    int cb_dt;
    SortedRot rot_h;
    SortedRot rot_i;
    void* out;
    int out_dt;
    int slices_gu;
    int slices_dn;
    void* workspace;
    size_t ws_bytes;
    void* stream;
};

size_t sorted_moe_workspace_bytes(int64_t n_pairs, int64_t hidden, int64_t inter, int slices_gu, int slices_dn);
int sorted_moe_launch(const SortedMoeCall& c);

// Device-resident expert pager (vq2_pager.hip).
size_t pager_lds_bytes(int64_t n_experts, int64_t capacity, int64_t n_pairs);
int pager_step_launch(const void* ids, int ids_i64, int64_t n_pairs, int64_t n_experts, int64_t capacity,
                      int32_t* slot_of, int32_t* expert_of, int32_t* stamp, int32_t* state, int32_t* copy_list,
                      int32_t* pair_slot, void* stream);
int pager_copy_launch(const void* mirror_host, int64_t record_bytes, const int64_t* seg_bytes, const int32_t* copy_list,
                      const int32_t* state, int64_t max_copies, void* const* dst, const int64_t* dst_stride,
                      int scale_dt, void* stream);

int rht_launch(const void* x, int x_dt, int64_t x_stride, void* y, int y_dt, int64_t y_stride,
               const int32_t* perm, const int8_t* sign, int64_t n, int64_t hb, int64_t batch, float scale,
               int inverse, int swiglu, int64_t inter, void* stream);

int argmax_launch(const void* v, int v_dt, int64_t rows, int64_t cols, int64_t* out_idx, float* out_val,
                  void* stream);

int router_launch(const void* logits, int l_dt, int64_t tokens, int64_t n_experts, int k, const void* h,
                  int h_dt, int64_t hidden, const void* gate, int g_dt, int64_t shared_id, int32_t* ids, float* w,
                  void* stream);

int dequant_launch(const int16_t* idx0, const void* idx1, int s2, const void* cb0, const void* cb1, int cb_dt,
                   const void* scale, int s_dt, int64_t r0, int64_t r1, int64_t n, float* out, void* stream);

int decode_launch(const void* in, int is_u8, int64_t count, int32_t* out, void* stream);

int unpack_fixed_launch(const uint8_t* buf, int64_t nbytes, int bits, int64_t n, int16_t* out, void* stream);

inline bool dt_ok(int dt) { return dt == VQ2_DT_F32 || dt == VQ2_DT_F16 || dt == VQ2_DT_BF16; }
inline int64_t dt_size(int dt) { return dt == VQ2_DT_F32 ? 4 : 2; }

}  // namespace vq2
