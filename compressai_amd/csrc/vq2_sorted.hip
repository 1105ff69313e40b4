// vq2_sorted.hip -- VQ GEMV over a code-sorted internal layout (gfx950).
//
//   y[r] = (sum_g cb0[i0[r, g]] . x_g  [+ sum_g cb1[i1[r, g]] . x_g]) * s[r] * rs
//
// Why: at batch 1 the reference layout costs one random 16-byte codebook
// gather per code, and random gathers from the L2-resident 1 MiB codebook are
// capped by the L2 request rate (about 240 G codes/s on MI355X, 6 % of HBM).
// Lanes whose codes fall in the same 128-byte codebook line share one
// request, so the codes of a chunk of rows are reordered by value: 64
// consecutive sorted codes of a chunk of ~65536 codes span about 8 lines
// instead of 64 (measured up to ~860 G codes/s for 65536-code chunks).
//
// Layout (built once at load time on the host by vq2_sorted_pack, from the
// reference's index planes, which stay the public format):
//  * a matrix is cut into chunks of R rows x all ng groups, gbits =
//    ceil(log2 ng) and R <= min(2^(17 - gbits) - 1, 511) rows (chosen at
//    pack time: the rows split evenly over the chunks; by default at most
//    min(2^(16 - gbits) - 1, 255), more for very tall matrices), so row R is
//    a dummy row that padding entries add to;
//  * every wave keeps two accumulator arrays, one per 32-lane half (four,
//    one per 16 lanes, for chunks of at most 32 rows of a dense matrix,
//    whose halves would otherwise run partly empty); a chunk's codes are
//    sorted by value (then position) and dealt into instructions of 64
//    lanes with no row twice in a lane group (an entry whose row every open
//    group already holds waits for the next instruction), so the lanes'
//    read-add-write of their row's accumulator never collide;
//  * lane 63 of an instruction carries its base code (the smallest), the
//    other 63 lanes one code each as a 24-bit field (code - base) << P | row
//    << gbits | group (P = gbits + bitlen(R) <= 17); an instruction whose next
//    code would be 2^(24 - P) or more above its base is closed early;
//    padding fills the tail;
//  * 4 instructions form an iteration of 768 bytes: lane l reads 12 bytes
//    (its four fields' low 16 bits in two words, their high bytes in a
//    third), so the entry stream is fully coalesced at 3 bytes per code;
//  * the chunk's stage-1 iterations come first, then its stage-2 iterations
//    (4 bpw), each stage padded to the matrix's largest count for it (ipc1,
//    ipc2), so chunk c holds iterations [c * ipc, (c + 1) * ipc), ipc = ipc1
//    + ipc2: a workgroup computes where its entries are from its chunk index
//    and issues their loads at once (a table of chunk offsets cost a memory
//    round trip in front of every other load).
//
// Kernel: one workgroup of 16 waves per (chunk, slice).  The workgroup first
// builds the rotated activation in LDS (the fused RHT prologue of the GEMV
// kernel, or a copy of a pre-rotated x), fp32; every wave owns two (or
// four) LDS accumulators per row of the chunk (parts x (R + 1) floats).  A
// wave takes iterations of its slice round-robin: one 12-byte entry load,
// four centroid gathers, then per entry the group's 8 activation values
// from LDS, the 8-term dot product in fp32 and acc[part][row] += dot.  At
// the end the waves' accumulators are summed in (wave, part) order: with one slice the rows are complete
// (y = (acc * s) * rs, or the fused top-1 key per workgroup); with several
// slices the raw partials go to a workspace and the last workgroup of the
// chunk to arrive sums them in slice order.  Every order is fixed, so results
// are deterministic.
//
// Semantics: vq_gemv_16 / the PackedLinear fallback (vq2/kernels.py:57-78,
// vq2/runtime.py:82-110) for the (16,) and (16,16) configurations; the sums
// are those of the gather kernels in another order (fp32 accumulation).
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "vq2_sorted.hpp"

namespace vq2 {


// Default chunk height: the rows split evenly over the fewest chunks of at
// most 255 rows with 16-bit positions; with chunk_align > 1, over a
// multiple of chunk_align chunks (one per CU and round: no CU waits for a
// last short round) when the chunks keep at least SG_MIN_ALIGNED_R rows.
// A matrix so tall that taller chunks (17-bit positions) fill a multiple of
// 2 x chunk_align chunks takes those: the LM head (151,936 rows) as 512
// chunks of 297 rows, one round of two workgroups per CU, instead of 768
// of 198 (measured 63.4 against 68.8 us per call).  More codes per chunk
// put more codes on each code value, so a wave's 63 sorted codes span
// fewer codebook lines.  (Taller chunks for the other shapes measured
// slower: gate+up 16.3 -> 17.5 us at 473 rows, down 13.8 -> 16.8 at 228.)
// With chunk_align > 1 a matrix of fewer than 2^20 codes takes about
// 0.75 x chunk_align chunks (at most 64 rows each), one workgroup each: its
// launch is bound by latency, and one slice per chunk saves the slice sum.
// Measured with 1024 HBM-resident copies, one slice: the o projection
// 2048 x 2048 at 11 / 16 / 20 / 24 / 32 rows 7.07 / 7.15 / 7.28 / 7.35 /
// 8.15 us (8.5 on the gather kernel, 9.0 at 9 chunks of 228 rows x 8
// slices); q, k and v in one launch, chunks from their total rows, at 16 /
// 24 / 32 rows 7.57 / 7.67 / 8.51 us (9.5 at 15 chunks of 171-228 rows x 8
// slices); fewer rows put the grid past one workgroup per CU (q, k, v at 12
// rows, 257 chunks: 10.1 us).
constexpr int64_t SG_MIN_ALIGNED_R = 128;
constexpr int64_t SG_SMALL_CODES = int64_t(1) << 20;
constexpr int64_t SG_SMALL_R = 64;
int64_t sorted_rows_per_chunk(int64_t out_rows, int64_t ng, int64_t chunk_align)
{
    const int64_t rmax = std::min<int64_t>(sorted_max_rows(ng, 16), 255);
    if (rmax == 0 || out_rows < 1) return 0;
    if (chunk_align > 1 && out_rows * ng < SG_SMALL_CODES) {
        const int64_t r = (4 * out_rows + 3 * chunk_align - 1) / (3 * chunk_align);
        return std::max<int64_t>(1, std::min(r, std::min(rmax, SG_SMALL_R)));
    }
    if (chunk_align > 1) {
        const int64_t rmax17 = sorted_max_rows(ng, 17), two = 2 * chunk_align;
        const int64_t n17 = ((out_rows + rmax17 - 1) / rmax17 + two - 1) / two * two;
        const int64_t r17 = (out_rows + n17 - 1) / n17;
        if (r17 > rmax) return r17;
    }
    const int64_t nch = (out_rows + rmax - 1) / rmax;
    if (chunk_align > 1) {
        const int64_t nal = (nch + chunk_align - 1) / chunk_align * chunk_align;
        const int64_t ral = (out_rows + nal - 1) / nal;
        if (ral >= SG_MIN_ALIGNED_R) return ral;
    }
    return (out_rows + nch - 1) / nch;
}

// ------------------------------------------------------------ host repack
// Whole iterations of padding: every field adds code 0 into the dummy row
// (position `pad`), the base lane's words hold base code 0.
static void fill_pad_iters(uint32_t* dst, int64_t iters, uint32_t pad)
{
    for (int64_t it = 0; it < iters; it++)
        for (int l = 0; l < 64; l++) {
            uint32_t* w = dst + (it * 64 + l) * SG_LANE_WORDS;
            // pad: up to 17 bits (its bit 16 in each field's high byte)
            const uint32_t pp = l == SG_BASE_LANE ? 0u : (pad & 0xFFFFu) | (pad & 0xFFFFu) << 16;
            w[0] = pp;
            w[1] = pp;
            w[2] = l == SG_BASE_LANE ? 0u : (pad >> 16) * 0x01010101u;
        }
}

// Entries of one (chunk, stage) in lane layout: sorted by code, dealt into
// 64-lane instructions (`parts` groups of 64 / parts lanes with distinct
// rows each: lanes 0-31 and 32-62, or 0-15, 16-31, 32-47 and 48-62; lane 63
// the instruction's base code) whose codes lie within 2^(24 - P) of the
// base, padded to whole iterations.
static void pack_chunk_stage(const int16_t* plane, int64_t r0, int64_t rows, int64_t ng, int gb, int64_t R,
                             int parts, std::vector<uint32_t>& out)
{
    const int pb = sorted_pbits(gb, (int)R);
    const uint32_t span = 1u << (24 - pb);  // code offsets below this
    // code << 32 | position (row << gb | group: up to 17 bits)
    std::vector<uint64_t> keys;
    keys.reserve((size_t)(rows * ng));
    for (int64_t r = 0; r < rows; r++) {
        const int16_t* p = plane + (r0 + r) * ng;
        for (int64_t g = 0; g < ng; g++)
            keys.push_back(((uint64_t)(uint16_t)p[g] << 32) | (uint64_t)((r << gb) | g));
    }
    std::sort(keys.begin(), keys.end());
    const uint32_t pad = (uint32_t)(R << gb);  // offset 0, dummy row R
    std::vector<uint32_t> instr;  // instruction-major 24-bit fields, 64 per instruction
    instr.reserve(keys.size() + keys.size() / 32 + 1024);
    std::vector<uint64_t> pending, still;
    // lane groups of the current instruction that hold each row (valid
    // while stamp[row] == id)
    std::vector<int64_t> stamp((size_t)R + 1, -1);
    std::vector<uint8_t> used((size_t)R + 1, 0);
    static_assert(SG_BASE_LANE == 63 && SG_MAX_PARTS <= 8, "the base in the last lane; one bit per part in used[]");
    const int pl = 64 / parts;  // lanes per part; the last part's last lane is the base
    int cap[SG_MAX_PARTS];
    for (int qd = 0; qd < parts; qd++) cap[qd] = qd + 1 < parts ? pl : pl - 1;
    size_t next = 0;
    int64_t id = 0;
    while (next < keys.size() || !pending.empty()) {
        uint32_t slot[SG_MAX_PARTS][64 / SG_PARTS];
        int fill[SG_MAX_PARTS] = {};
        int n = 0;
        bool have_base = false;
        uint32_t base = 0;
        // place k in the first open lane group that does not hold its row:
        // 0 placed, 1 its row is in both groups, 2 its code is too far from
        // the base (every later key's is too: codes ascend)
        auto place = [&](uint64_t k) -> int {
            const uint32_t code = (uint32_t)(k >> 32), kp = (uint32_t)k;
            if (have_base && code - base >= span) return 2;
            const uint32_t row = kp >> gb;
            const uint8_t u = stamp[row] == id ? used[row] : 0;
            for (int qd = 0; qd < parts; qd++)
                if (fill[qd] < cap[qd] && !(u & (1u << qd))) {
                    if (!have_base) {
                        have_base = true;
                        base = code;
                    }
                    slot[qd][fill[qd]++] = ((code - base) << pb) | kp;
                    stamp[row] = id;
                    used[row] = (uint8_t)(u | (1u << qd));
                    n++;
                    return 0;
                }
            return 1;
        };
        const int full = 63;
        // entries waiting since an earlier instruction go first (their codes
        // are the smallest left, in ascending order, so the first one placed
        // is the instruction's smallest code)
        still.clear();
        size_t i = 0;
        for (; i < pending.size() && n < full; i++) {
            const int r = place(pending[i]);
            if (r == 2) break;
            if (r == 1) still.push_back(pending[i]);
        }
        const bool closed = i < pending.size() && n < full;
        for (; i < pending.size(); i++) still.push_back(pending[i]);
        pending.swap(still);
        while (!closed && n < full && next < keys.size()) {
            const int r = place(keys[next]);
            if (r == 2) break;
            if (r == 1) pending.push_back(keys[next]);
            next++;
        }
        for (int qd = 0; qd < parts; qd++) {
            while (fill[qd] < pl) slot[qd][fill[qd]++] = pad;
            instr.insert(instr.end(), slot[qd], slot[qd] + pl);
        }
        instr.back() = base;  // lane 63: the base code
        id++;
    }
    while ((instr.size() / 64) % 4) {
        instr.insert(instr.end(), 64, pad);
        instr.back() = 0u;
    }
    const size_t iters = instr.size() / SG_ITER;
    const size_t at = out.size();
    out.resize(at + iters * SG_ITER_WORDS);
    for (size_t it = 0; it < iters; it++)
        for (int l = 0; l < 64; l++) {
            uint32_t f[4];
            for (int q = 0; q < 4; q++) f[q] = instr[(it * 4 + q) * 64 + l];
            uint32_t* w = &out[at + (it * 64 + l) * SG_LANE_WORDS];
            w[0] = (f[0] & 0xFFFFu) | (f[1] & 0xFFFFu) << 16;
            w[1] = (f[2] & 0xFFFFu) | (f[3] & 0xFFFFu) << 16;
            w[2] = (f[0] >> 16) | (f[1] >> 16) << 8 | (f[2] >> 16) << 16 | (f[3] >> 16) << 24;
        }
}

int sorted_pack(const int16_t* idx0, const int16_t* idx1, int64_t out_rows, int64_t ng, int64_t R,
                uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk, int64_t* stage1_iters,
                int64_t* n_iters, int n_threads)
{
    const int64_t rmax = sorted_max_rows(ng);
    if (rmax == 0) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_pack: ng=%lld outside 1..32768", (long long)ng);
    if (R < 1 || R > rmax)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_pack: rows_per_chunk=%lld outside 1..%lld for ng=%lld",
                         (long long)R, (long long)rmax, (long long)ng);
    const int gb = sorted_gbits(ng);
    const ChunkSplit ks = chunk_split(out_rows, R);
    const int64_t n_chunks = ks.n_chunks;
    std::vector<std::vector<uint32_t>> p1((size_t)n_chunks), p2((size_t)n_chunks);
    int nt = n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency();
    if (nt < 1) nt = 1;
    if (nt > n_chunks) nt = (int)(n_chunks > 0 ? n_chunks : 1);
    auto work = [&](int t) {
        for (int64_t c = t; c < n_chunks; c += nt) {
            const int64_t r0 = c * ks.rb + std::min(c, ks.nbig), rows = ks.rb + (c < ks.nbig ? 1 : 0);
            pack_chunk_stage(idx0, r0, rows, ng, gb, R, sorted_parts(R), p1[c]);
            if (idx1) pack_chunk_stage(idx1, r0, rows, ng, gb, R, sorted_parts(R), p2[c]);
        }
    };
    if (nt == 1) {
        work(0);
    } else {
        std::vector<std::thread> th;
        for (int t = 0; t < nt; t++) th.emplace_back(work, t);
        for (auto& t : th) t.join();
    }
    // every chunk's stages padded to the largest stage-1 / stage-2 iteration
    // counts, so chunk c holds iterations [c * ipc, (c + 1) * ipc) with its
    // stage-2 entries from c * ipc + ipc1 on: a workgroup computes where its
    // entries are instead of reading a table
    int64_t ipc1 = 0, ipc2 = 0;
    for (int64_t c = 0; c < n_chunks; c++) {
        ipc1 = std::max(ipc1, (int64_t)p1[c].size() / SG_ITER_WORDS);
        ipc2 = std::max(ipc2, (int64_t)p2[c].size() / SG_ITER_WORDS);
    }
    const int64_t ipc = ipc1 + ipc2;
    const int64_t total = ipc * n_chunks;
    *n_iters = total;
    *iters_per_chunk = ipc;
    *stage1_iters = ipc1;
    if (total > 0x7FFFFFFFLL) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_pack: matrix too large");
    if (total > cap_iters)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_pack: %lld iterations needed, capacity %lld", (long long)total,
                         (long long)cap_iters);
    const uint32_t pad = (uint32_t)(R << gb);  // code 0, dummy row R
    for (int64_t c = 0; c < n_chunks; c++) {
        uint32_t* d1 = entries + c * ipc * SG_ITER_WORDS;
        uint32_t* d2 = d1 + ipc1 * SG_ITER_WORDS;
        const int64_t n1 = (int64_t)p1[c].size() / SG_ITER_WORDS, n2 = (int64_t)p2[c].size() / SG_ITER_WORDS;
        memcpy(d1, p1[c].data(), p1[c].size() * sizeof(uint32_t));
        fill_pad_iters(d1 + n1 * SG_ITER_WORDS, ipc1 - n1, pad);
        memcpy(d2, p2[c].data(), p2[c].size() * sizeof(uint32_t));
        fill_pad_iters(d2 + n2 * SG_ITER_WORDS, ipc2 - n2, pad);
    }
    return VQ2_OK;
}

// Expert pool [E, rows, ng] (one or two stages): every expert packed as a
// matrix of its own with the same chunk height R, experts one after another,
// and every chunk's stage-1 and stage-2 entries padded (dummy-row entries)
// to the pool's largest stage-1 / stage-2 iteration counts, so chunk c of
// expert e starts at iteration (e * C + c) * ipc (C = ceil(rows / R)), its
// stage-2 entries ipc1 later, with no table to read.
int sorted_pack_pool(const int16_t* idx, const int16_t* idx1, int64_t n_experts, int64_t rows, int64_t ng, int64_t R,
                     uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk, int64_t* stage1_iters,
                     int64_t* n_iters, int n_threads)
{
    const int64_t rmax = sorted_max_rows(ng, 16);  // pools: 16-bit positions
    if (rmax == 0) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_pack_pool: ng=%lld outside 1..32768", (long long)ng);
    if (R < 1 || R > rmax)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_pack_pool: rows_per_chunk=%lld outside 1..%lld for ng=%lld",
                         (long long)R, (long long)rmax, (long long)ng);
    const int gb = sorted_gbits(ng);
    const ChunkSplit ks = chunk_split(rows, R);
    const int64_t C = ks.n_chunks;
    const int64_t units = n_experts * C;
    std::vector<std::vector<uint32_t>> p1((size_t)units), p2((size_t)units);
    int nt = n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency();
    if (nt < 1) nt = 1;
    if (nt > units) nt = (int)(units > 0 ? units : 1);
    auto work = [&](int t) {
        for (int64_t u = t; u < units; u += nt) {
            const int64_t e = u / C, c = u - e * C;
            const int64_t r0 = c * ks.rb + std::min(c, ks.nbig), nr = ks.rb + (c < ks.nbig ? 1 : 0);
            pack_chunk_stage(idx + e * rows * ng, r0, nr, ng, gb, R, SG_PARTS, p1[u]);
            if (idx1) pack_chunk_stage(idx1 + e * rows * ng, r0, nr, ng, gb, R, SG_PARTS, p2[u]);
        }
    };
    if (nt == 1) {
        work(0);
    } else {
        std::vector<std::thread> th;
        for (int t = 0; t < nt; t++) th.emplace_back(work, t);
        for (auto& t : th) t.join();
    }
    int64_t ipc1 = 1, ipc2 = 0;
    for (int64_t u = 0; u < units; u++) {
        ipc1 = std::max(ipc1, (int64_t)p1[u].size() / SG_ITER_WORDS);
        ipc2 = std::max(ipc2, (int64_t)p2[u].size() / SG_ITER_WORDS);
    }
    const int64_t ipc = ipc1 + ipc2;
    const int64_t total = ipc * units;
    *n_iters = total;
    *iters_per_chunk = ipc;
    *stage1_iters = ipc1;
    if (total > 0x7FFFFFFFLL) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_pack_pool: pool too large");
    if (total > cap_iters)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_pack_pool: %lld iterations needed, capacity %lld", (long long)total,
                         (long long)cap_iters);
    const uint32_t pad = (uint32_t)(R << gb);  // code 0, dummy row R
    for (int64_t u = 0; u < units; u++) {
        uint32_t* d1 = entries + u * ipc * SG_ITER_WORDS;
        uint32_t* d2 = d1 + ipc1 * SG_ITER_WORDS;
        const int64_t n1 = (int64_t)p1[u].size() / SG_ITER_WORDS, n2 = (int64_t)p2[u].size() / SG_ITER_WORDS;
        memcpy(d1, p1[u].data(), p1[u].size() * sizeof(uint32_t));
        fill_pad_iters(d1 + n1 * SG_ITER_WORDS, ipc1 - n1, pad);
        memcpy(d2, p2[u].data(), p2[u].size() * sizeof(uint32_t));
        fill_pad_iters(d2 + n2 * SG_ITER_WORDS, ipc2 - n2, pad);
    }
    return VQ2_OK;
}

// ------------------------------------------------------------------ kernel
struct SortedSeg {
    const uint32_t* ent;  // [n_iters * SG_ITER_WORDS] lane words
    int32_t ipc;       // iterations per chunk (chunk c: [c * ipc, (c + 1) * ipc))
    int32_t ipc1;      // its stage-1 iterations (the stage-2 ones follow)
    const void* scale;
    void* y;
    float* part;    // slices > 1: [slices][out_rows] raw row sums
    uint32_t* cnt;  // slices > 1: arrival counter per chunk
    int64_t out_rows;
    int32_t n_iters;
    int32_t n_chunks;
    int32_t chunk_start;  // the matrix's first chunk in the launch's chunk numbering
    int32_t sq, sr;       // slice j of a chunk: sq + (j < sr) iterations, from j * sq + min(j, sr)
    int32_t R;     // rows per chunk at most (row R is the dummy row)
    int32_t rb;    // chunk c: rows [c * rb + min(c, nbig), + rb + (c < nbig))
    int32_t nbig;
};

struct SortedArgs {
    GemvArgs g;  // the activation fields of the prologue (x, perm, sign, hb_log2, xscale, strides)
    const void* cb0;
    const void* cb1;
    uint32_t c1mask;  // stage-2 code mask (0xFF: the 256-row codebook of (16,8))
    int s_dt;
    int y_dt;
    int64_t ng;
    int gbits;
    int slices;
    float rs;
    int nseg;
    int nc;          // chunks over all matrices
    SortedSeg seg[SG_MAX_SEG];
    uint64_t* cand;  // EP 1: best top-1 key per workgroup
};

// XM 0: x holds the rotated activation (dtype XT); XM 1: rotate x in LDS.
// EP 0: store y (or partials with several slices); EP 1: fused top-1 keys.
// The fused-RHT top-1 (the LM head: 768 workgroups, three per CU) is held
// to 64 VGPRs so that two workgroups share a CU and one's prologue overlaps
// the other's gathers (measured 72.5 against 77.8 us at 70 VGPRs); the
// other instantiations run one workgroup per CU, where that bound only
// costs spills (gate+up 19.1 -> 20.0 us).
//
// What the first loads need comes first as 14 dwords of scalar kernel
// arguments: with -amdgpu-kernarg-preload-count the wave starts with them in
// SGPRs, so the activation, permutation and sign loads and the first entry
// words of a workgroup of the first two matrices issue at once, not after a
// load of the argument lines (dense step 45.94 -> 45.64 us with the
// activation fields alone).  k_ent0 / k_ent1: the entries of matrices 0 and
// 1 (matrix 0 twice in a one-matrix launch); k_geo0 / k_geo1: their
// iterations per chunk | iterations per slice << 16; k_cs: chunks over all
// matrices | matrix 1's first chunk << 16 (the chunk count itself in a
// one-matrix launch); k_srn: the two matrices' longer-slice counts (8 bits
// each) | matrix count << 16 | 2048-point blocks of the activation << 24.
// TALL: a launch whose chunks hold 256 or more rows or 17-bit positions
// (very tall matrices: the LM head); it also keeps the split activation in
// n floats (halves n / 2 apart) so that the LM head's workgroups stay
// small enough for two per CU; the other instantiations keep SG_XB.
template <int CBT, int XM, int XT, int EP, bool TALL>
__global__ void __launch_bounds__(SG_THREADS, (XM != 0 && EP == 1) ? 8 : 1)
    vq_sorted_kernel(const void* const k_x, const int32_t* const k_perm, const int8_t* const k_sign,
                     const uint32_t* const k_ent0, const uint32_t* const k_ent1, const uint32_t k_geo0,
                     const uint32_t k_geo1, const uint32_t k_cs, const uint32_t k_srn, const SortedArgs a)
{
    extern __shared__ __align__(16) float smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // the 2048-point block count (XM 3) from the leading arguments: a.ng
    // would be a load of the argument struct ahead of the first loads
    const int k2k = (int)(k_srn >> 24);
    const int64_t n = XM == 3 ? (int64_t)k2k * RHT2K : a.ng * 8;
    // XM 1 / 3: [natural-order activation: n][stage (n), later the split
    // activation (SG_X_SPLIT floats, or TALL: n floats)][accumulators]; XM 0:
    // [split][accumulators]
    float* s_nat = smem;
    const int xb = TALL ? (int)(n / 2) : SG_XB;
    float* s_x = smem + (XM != 0 ? n : 0);              // split activation
    float* s_acc = s_x + (TALL ? n : SG_X_SPLIT);       // SG_WAVES x sorted_parts(R) x (R + 1)
    // prologue loads first (they need only the activation fields, and
    // return before the entries and gathers)
    XProLoad first;
    Rht2kLoad first2k;
    const int64_t t0 = (int64_t)threadIdx.x * 8;
    if constexpr (XM == 1) xpro_load<1, XT>(a.g, t0 < n ? t0 : 0, n, 0, 0, first);
    if constexpr (XM == 3) rht2k_load<XT>(k_x, k_perm, k_sign, k2k, 0, first2k);

    // workgroup b: slice b / nc of chunk b % nc (over all matrices); the
    // slice bounds come from the host (no divisions ahead of the entry
    // loads: with them and the prologue loads issued after the segment
    // lookup, gate+up took 16.8 us, 15.9 us without).  Matrices 0 and 1
    // from the leading arguments, 2 and 3 from the argument struct.
    const int nc = (int)(k_cs & 0xFFFFu), cs1 = (int)(k_cs >> 16);
    const int nseg = (int)((k_srn >> 16) & 0xFFu);
    const int pos = (int)blockIdx.x;
    const int slice = pos / nc, gchunk = pos - slice * nc;
    int si = gchunk < cs1 ? 0 : 1;
    const uint32_t geo = si == 0 ? k_geo0 : k_geo1;
    const uint32_t* ent = si == 0 ? k_ent0 : k_ent1;
    int ipc = (int)(geo & 0xFFFFu), sq = (int)(geo >> 16), sr = (int)((k_srn >> (8 * si)) & 0xFFu);
    int chunk = gchunk - (si == 0 ? 0 : cs1);
    if (si == 1 && nseg > 2) {
#pragma unroll
        for (int s = 2; s < SG_MAX_SEG; s++) si += (s < nseg && gchunk >= a.seg[s].chunk_start) ? 1 : 0;
        if (si > 1) {
            ent = a.seg[si].ent;
            ipc = a.seg[si].ipc;
            sq = a.seg[si].sq;
            sr = a.seg[si].sr;
            chunk = gchunk - a.seg[si].chunk_start;
        }
        // the wait for these scalar loads stays on this path (merged after
        // the branch, it held every workgroup's entry loads behind the
        // argument struct's other loads)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    }
    // chunk < n_chunks and n_iters = n_chunks * ipc (checked on the host)
    const int c_beg = chunk * ipc;
    const int s0 = c_beg + slice * sq + min(slice, sr);
    const int s1 = s0 + sq + (slice < sr ? 1 : 0);

    // the wave's first entry words come from HBM while the prologue stages
    // and rotates the activation (which waits only for its own, earlier
    // loads); the first gathers go out inside it (XM 3) or after it (XM 1)
    // (a pre-rotated x is only copied: there the gathers go out at once)
    // gathers one iteration ahead (measured on the dense step: 49.1 us
    // against 49.3 at two; three, before the pipeline's tail stopped loading
    // past the range, 51.3 against 50.2 at two; with 3-byte entries and the
    // leading arguments 42.2 against 45.5 at two); the top-1 of the LM head
    // too, two workgroups per CU (pre-rotated: 51.5 against 55.6 us at two)
    SortedPipe<CBT, 1, SG_WAVES, TALL> pipe;
    pipe.load_entries(ent, a.cb0, a.cb1, c_beg, c_beg, s0, s1, wave, lane, 0, 1, a.c1mask);
    // the fields the loop needs, from the argument struct (its lines were
    // not needed before this point)
    touch_kernargs(a);
    const SortedSeg& sg = a.seg[si];
    const int R = sg.R;
    pipe.set_fields(c_beg + sg.ipc1, a.gbits, R);
    if constexpr (XM == 0) pipe.gathers();

    const int parts = sorted_parts(R);
    float* acc = sorted_acc(s_acc, wave, lane, R, parts);
    sorted_acc_zero(acc, lane, R, parts);
    if constexpr (XM == 1) {
        void* s_stage = smem + n;  // dead once build_x is done: the split activation takes its place
        stage_x<1, XT>(a.g, s_stage, 1, n, 0, 0, first);
        build_x<1, XT>(a.g, s_nat, s_stage, 1, n, first);
        x_finalize(s_nat, s_x, n, a.g.xscale, xb);
    } else if constexpr (XM == 3) {
        // the first gathers go out between the lane stages and the LDS
        // passes (measured: dense step 46.96 -> 46.65 us, LM head 65.2 ->
        // 64.9; before the transform, waiting there for the entry words:
        // 48.1)
        rht2k_build<XT>(k2k, n, first2k, smem + n, s_nat, s_x, a.g.xscale, xb, [&]() { pipe.gathers(); });
    } else {
        for (int64_t g = threadIdx.x; g < a.ng; g += SG_THREADS) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = load_as_f32(a.g.x, XT, g * 8 + k);
            x_store_group(s_x, g, v, xb);
        }
    }
    __syncthreads();
    if constexpr (XM == 1) pipe.gathers();
    pipe.run(acc, s_x, a.gbits, a.ng, R, xb);
    __syncthreads();

    __shared__ float s_red[4][256];
    const float sum = sorted_row_sums<TALL>(s_acc, R, s_red, parts);
    // thread rr < R holds row rr's sum
    const int rr = TALL ? (int)threadIdx.x : (int)(threadIdx.x & 255);
    const bool lead = TALL || threadIdx.x < 256;
    const int64_t row0 = (int64_t)chunk * sg.rb + min(chunk, sg.nbig);
    const int64_t row = row0 + rr;
    const bool own = lead && rr < sg.rb + (chunk < sg.nbig ? 1 : 0);
    if constexpr (EP == 1) {
        uint64_t best = own ? argmax_key((sum * load_as_f32(sg.scale, a.s_dt, row)) * a.rs, row) : 0;
        for (int off = 32; off > 0; off >>= 1) {
            const uint64_t o = __shfl_xor(best, off);
            best = o > best ? o : best;
        }
        // the rows are the first 4 waves' threads (TALL: 8, at most 511 rows)
        constexpr int KW = TALL ? 8 : 4;
        __shared__ uint64_t s_key[KW];
        if (wave < KW && lane == 0) s_key[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < KW; w++) best = s_key[w] > best ? s_key[w] : best;
            a.cand[blockIdx.x] = best;
        }
    } else if (a.slices == 1) {
        if (own) store_from_f32(sg.y, a.y_dt, row, (sum * load_as_f32(sg.scale, a.s_dt, row)) * a.rs);
    } else {
        // several slices: the last of the chunk's workgroups to finish adds
        // the slices' raw row sums in slice order
        if (own) share_store(sg.part + (int64_t)slice * sg.out_rows + row, sum);
        if (arrive_last(sg.cnt + chunk, (uint32_t)a.slices) && own) {
            float tot = 0.0f;
            for (int s0 = 0; s0 < a.slices; s0 += 8) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int s = s0 + j < a.slices ? s0 + j : slice;
                    v[j] = s == slice ? sum : share_load(sg.part + (int64_t)s * sg.out_rows + row);
                }
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (s0 + j < a.slices) tot += v[j];
            }
            store_from_f32(sg.y, a.y_dt, row, (tot * load_as_f32(sg.scale, a.s_dt, row)) * a.rs);
        }
    }
}

// ------------------------------------------------------------------ launch
template <int CBT, int XM, int XT, int EP, bool TALL>
static hipError_t launch_sorted(const SortedArgs& a, unsigned grid, size_t shm, hipStream_t st)
{
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)vq_sorted_kernel<CBT, XM, XT, EP, TALL>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, SG_MAX_SHM);
    });
    if (attr != hipSuccess) return attr;
    // the leading arguments: matrices 0 and 1 (matrix 0 again for a
    // one-matrix launch, whose chunks all lie below cs1 = nc)
    const SortedSeg& s0 = a.seg[0];
    const SortedSeg& s1 = a.seg[a.nseg > 1 ? 1 : 0];
    const uint32_t geo0 = (uint32_t)s0.ipc | (uint32_t)s0.sq << 16, geo1 = (uint32_t)s1.ipc | (uint32_t)s1.sq << 16;
    const uint32_t cs = (uint32_t)a.nc | (uint32_t)(a.nseg > 1 ? s1.chunk_start : a.nc) << 16;
    const uint32_t srn = (uint32_t)s0.sr | (uint32_t)s1.sr << 8 | (uint32_t)a.nseg << 16 |
                         (uint32_t)(a.ng * 8 / RHT2K) << 24;
    hipLaunchKernelGGL((vq_sorted_kernel<CBT, XM, XT, EP, TALL>), dim3(grid), dim3(SG_THREADS), shm, st, a.g.x,
                       a.g.perm, a.g.sign, s0.ent, s1.ent, geo0, geo1, cs, srn, a);
    return hipGetLastError();
}

// TALL launches: the 2048-point prologue (XM 3) or a rotated activation
// (XM 0) only (the host refuses the others)
template <int CBT, int EP, bool TALL>
static hipError_t launch_sorted_t(int xm, int x_dt, const SortedArgs& a, unsigned grid, size_t shm, hipStream_t st)
{
    if (xm == 3) {
        switch (x_dt) {
        case VQ2_DT_F16: return launch_sorted<CBT, 3, VQ2_DT_F16, EP, TALL>(a, grid, shm, st);
        case VQ2_DT_BF16: return launch_sorted<CBT, 3, VQ2_DT_BF16, EP, TALL>(a, grid, shm, st);
        default: return launch_sorted<CBT, 3, VQ2_DT_F32, EP, TALL>(a, grid, shm, st);
        }
    }
    if constexpr (!TALL) {
        if (xm == 1) {
            switch (x_dt) {
            case VQ2_DT_F16: return launch_sorted<CBT, 1, VQ2_DT_F16, EP, false>(a, grid, shm, st);
            case VQ2_DT_BF16: return launch_sorted<CBT, 1, VQ2_DT_BF16, EP, false>(a, grid, shm, st);
            default: return launch_sorted<CBT, 1, VQ2_DT_F32, EP, false>(a, grid, shm, st);
            }
        }
    } else if (xm == 1) {
        return hipErrorInvalidValue;
    }
    switch (x_dt) {
    case VQ2_DT_F16: return launch_sorted<CBT, 0, VQ2_DT_F16, EP, TALL>(a, grid, shm, st);
    case VQ2_DT_BF16: return launch_sorted<CBT, 0, VQ2_DT_BF16, EP, TALL>(a, grid, shm, st);
    default: return launch_sorted<CBT, 0, VQ2_DT_F32, EP, TALL>(a, grid, shm, st);
    }
}

template <int CBT, int EP>
static hipError_t launch_sorted_x(int xm, int x_dt, bool tall, const SortedArgs& a, unsigned grid, size_t shm,
                                  hipStream_t st)
{
    return tall ? launch_sorted_t<CBT, EP, true>(xm, x_dt, a, grid, shm, st)
                : launch_sorted_t<CBT, EP, false>(xm, x_dt, a, grid, shm, st);
}

// Workspace with several slices: VQ2_SORTED_WS_HEADER bytes of arrival
// counters (zero between launches), then the slices' raw row sums (matrix
// after matrix).  Top-1: one key per workgroup.
size_t sorted_workspace_bytes(const SortedCall& c)
{
    if (c.slices <= 1) return 0;
    size_t b = VQ2_SORTED_WS_HEADER;
    for (int s = 0; s < c.nseg; s++) b += (size_t)c.slices * c.seg[s].out_rows * sizeof(float);
    return b;
}

size_t sorted_top1_workspace_bytes(int64_t out_rows, int64_t rows_per_chunk)
{
    if (rows_per_chunk < 1 || out_rows < 1) return 0;
    return (size_t)((out_rows + rows_per_chunk - 1) / rows_per_chunk) * sizeof(uint64_t);
}

int64_t sorted_acc_arrays(const SortedCall& c)
{
    int64_t f = 0;
    for (int s = 0; s < c.nseg; s++) {
        const int64_t R = c.seg[s].rows_per_chunk;
        f = std::max<int64_t>(f, sorted_parts(R) * (R + 1));
    }
    return f;
}

int sorted_check_call(const SortedCall& c, bool top1, const char* who, int64_t* rmax)
{
    if (c.nseg < 1 || c.nseg > SG_MAX_SEG) return set_error(VQ2_ERR_ARG, "%s: 1..%d matrices", who, SG_MAX_SEG);
    const int64_t r_lim = sorted_max_rows(c.ng);
    if (r_lim == 0) return set_error(VQ2_ERR_UNSUPPORTED, "%s: ng=%lld unsupported", who, (long long)c.ng);
    *rmax = 0;
    for (int s = 0; s < c.nseg; s++) {
        const int64_t R = c.seg[s].rows_per_chunk;
        if (R < 1 || R > r_lim)
            return set_error(VQ2_ERR_ARG, "%s: matrix %d: rows_per_chunk=%lld outside 1..%lld", who, s, (long long)R,
                             (long long)r_lim);
        *rmax = std::max(*rmax, R);
    }
    if (c.cb_dt != VQ2_DT_F16 && c.cb_dt != VQ2_DT_BF16)
        return set_error(VQ2_ERR_UNSUPPORTED, "%s: fp16 / bf16 codebooks only", who);
    if (c.slices < 1 || c.slices > 64) return set_error(VQ2_ERR_ARG, "%s: slices must be 1..64", who);
    if (top1 && (c.slices != 1 || c.nseg != 1)) return set_error(VQ2_ERR_ARG, "%s top-1: one matrix, one slice", who);
    if ((uintptr_t)c.cb0 % 16 || (c.cb1 && (uintptr_t)c.cb1 % 16))
        return set_error(VQ2_ERR_ARG, "%s: codebooks must be 16-byte aligned", who);
    return VQ2_OK;
}

int sorted_check_seg(const SortedCall& c, int s, const char* who, ChunkSplit* ks)
{
    const SortedSegCall& sc = c.seg[s];
    *ks = chunk_split(sc.out_rows, sc.rows_per_chunk);
    if (sc.n_iters < 1 || sc.n_iters > 0x7FFFFFFF)
        return set_error(VQ2_ERR_ARG, "%s: matrix %d has %lld iterations", who, s, (long long)sc.n_iters);
    if ((uintptr_t)sc.entries % 16) return set_error(VQ2_ERR_ARG, "%s: entries must be 16-byte aligned", who);
    if (sc.s2 != (c.cb1 != nullptr)) return set_error(VQ2_ERR_ARG, "%s: stage-2 entries need cb1", who);
    if (sc.iters_per_chunk < 1 || sc.stage1_iters < 0 || sc.stage1_iters > sc.iters_per_chunk ||
        sc.iters_per_chunk * ks->n_chunks != sc.n_iters || (!sc.s2 && sc.stage1_iters != sc.iters_per_chunk))
        return set_error(VQ2_ERR_ARG, "%s: matrix %d: %lld iterations are not %lld chunks x %lld (%lld of stage 1)",
                         who, s, (long long)sc.n_iters, (long long)ks->n_chunks, (long long)sc.iters_per_chunk,
                         (long long)sc.stage1_iters);
    return VQ2_OK;
}

int sorted_launch(const SortedCall& c, int64_t* top1_idx, float* top1_val)
{
    const bool top1 = top1_idx != nullptr;
    int64_t rmax = 0;
    if (int r = sorted_check_call(c, top1, "vq2 sorted GEMV", &rmax)) return r;
    const int64_t n = c.ng * 8;
    // chunks of 256 rows or more, or 17-bit positions: the TALL kernels
    const bool tall = rmax >= 256 || sorted_pbits(sorted_gbits(c.ng), (int)rmax) > 16;
    const size_t shm =
        (size_t)((c.xm != 0 ? n : 0) + (tall ? n : SG_X_SPLIT) + SG_WAVES * sorted_acc_arrays(c)) * sizeof(float);
    if (n > 2 * SG_XB || shm > SG_MAX_SHM)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: n=%lld too large (at most %d)", (long long)n, 2 * SG_XB);
    if (c.xm == 1) {
        if (n % 64) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: fused RHT needs n %% 64 == 0");
        if (c.hb < 2 || c.hb > n || (c.hb & (c.hb - 1)) || n % c.hb)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMV: hb=%lld must be a power of two dividing n", (long long)c.hb);
        if ((uintptr_t)c.perm % 16 || (uintptr_t)c.sign % 8)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMV: perm 16-byte, sign 8-byte aligned");
        if ((uintptr_t)c.x % 16) return set_error(VQ2_ERR_ARG, "vq2 sorted GEMV: x must be 16-byte aligned");
    }
    // 2048-point blocks: the all-threads prologue (rht2k_build)
    const int xm = (c.xm == 1 && c.hb == RHT2K && n % RHT2K == 0 && n <= (int64_t)RHT2K * RHT2K_MAXB) ? 3 : c.xm;
    if (tall && xm == 1)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: chunks of %lld rows (256 or more, or 17-bit positions) "
                         "need a 2048-point rotation or a rotated activation", (long long)rmax);
    SortedArgs a{};
    a.g.x = c.x;
    a.g.x_dt = c.x_dt;
    a.g.x_bstride = n;
    a.g.x_pstride = 0;
    a.g.x_pdiv = 1;
    a.g.P = 1;
    a.g.ng = c.ng;
    a.g.batch = 1;
    a.g.perm = c.perm;
    a.g.sign = c.sign;
    int hl = 0;
    while ((int64_t(1) << hl) < c.hb) hl++;
    a.g.hb_log2 = hl;
    a.g.xscale = c.xscale;
    a.cb0 = c.cb0;
    a.cb1 = c.cb1;
    a.c1mask = c.cb1_rows == 256 ? 0xFFu : 0xFFFFu;
    a.s_dt = c.s_dt;
    a.y_dt = c.y_dt;
    a.ng = c.ng;
    a.gbits = sorted_gbits(c.ng);
    a.slices = c.slices;
    a.rs = c.rs;
    a.nseg = c.nseg;
    uint32_t* cnt = (uint32_t*)c.workspace;
    float* part = (float*)((char*)c.workspace + VQ2_SORTED_WS_HEADER);
    if (top1) {
        const size_t need = sorted_top1_workspace_bytes(c.seg[0].out_rows, c.seg[0].rows_per_chunk);
        if (!c.workspace || c.ws_bytes < need || (uintptr_t)c.workspace % 8)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMV top-1: workspace of %zu bytes (8-byte aligned) needed, got "
                             "%zu", need, c.ws_bytes);
        a.cand = (uint64_t*)c.workspace;
    } else if (c.slices > 1) {
        const size_t need = sorted_workspace_bytes(c);
        if (!c.workspace || c.ws_bytes < need || (uintptr_t)c.workspace % 16)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMV: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                             need, c.ws_bytes);
    }
    int64_t wg = 0, n_cnt = 0, nc = 0;
    for (int s = 0; s < c.nseg; s++) {
        const SortedSegCall& sc = c.seg[s];
        const int64_t R = sc.rows_per_chunk;
        ChunkSplit ks;
        if (int r = sorted_check_seg(c, s, "vq2 sorted GEMV", &ks)) return r;
        const int64_t n_chunks = ks.n_chunks;
        a.seg[s].ent = sc.entries;
        a.seg[s].ipc = (int32_t)sc.iters_per_chunk;
        a.seg[s].ipc1 = (int32_t)sc.stage1_iters;
        a.seg[s].scale = sc.scale;
        a.seg[s].y = sc.y;
        a.seg[s].out_rows = sc.out_rows;
        a.seg[s].n_iters = (int32_t)sc.n_iters;
        a.seg[s].n_chunks = (int32_t)n_chunks;
        a.seg[s].chunk_start = (int32_t)nc;
        a.seg[s].sq = (int32_t)(sc.iters_per_chunk / c.slices);
        a.seg[s].sr = (int32_t)(sc.iters_per_chunk % c.slices);
        a.seg[s].R = (int32_t)R;
        a.seg[s].rb = (int32_t)ks.rb;
        a.seg[s].nbig = (int32_t)ks.nbig;
        a.seg[s].part = part;
        a.seg[s].cnt = cnt + n_cnt;
        if (!top1 && c.slices > 1) {
            part += c.slices * sc.out_rows;
            n_cnt += n_chunks;
        }
        wg += n_chunks * c.slices;
        nc += n_chunks;
    }
    if (n_cnt > VQ2_SORTED_MAX_COUNTERS)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: %lld chunks with several slices (at most %d)",
                         (long long)n_cnt, VQ2_SORTED_MAX_COUNTERS);
    if (wg == 0) return VQ2_OK;
    if (wg > 0x7FFFFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: grid too large");
    // the leading kernel arguments carry chunk counts, iterations per chunk
    // and slice lengths in 16 bits
    if (nc > 0xFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: %lld chunks (at most 65535)", (long long)nc);
    for (int s = 0; s < c.nseg; s++)
        if (c.seg[s].iters_per_chunk > 0xFFFF)
            return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMV: matrix %d: %lld iterations per chunk (at most "
                             "65535)", s, (long long)c.seg[s].iters_per_chunk);
    a.nc = (int)nc;
    hipStream_t st = (hipStream_t)c.stream;
    hipError_t err;
    if (top1) {
        err = c.cb_dt == VQ2_DT_F16 ? launch_sorted_x<VQ2_DT_F16, 1>(xm, c.x_dt, tall, a, (unsigned)wg, shm, st)
                                    : launch_sorted_x<VQ2_DT_BF16, 1>(xm, c.x_dt, tall, a, (unsigned)wg, shm, st);
        if (err != hipSuccess) return set_hip_error(err, "vq2 sorted GEMV launch");
        return argmax_final_launch(a.cand, wg, 1, top1_idx, top1_val, c.stream);
    }
    err = c.cb_dt == VQ2_DT_F16 ? launch_sorted_x<VQ2_DT_F16, 0>(xm, c.x_dt, tall, a, (unsigned)wg, shm, st)
                                : launch_sorted_x<VQ2_DT_BF16, 0>(xm, c.x_dt, tall, a, (unsigned)wg, shm, st);
    if (err != hipSuccess) return set_hip_error(err, "vq2 sorted GEMV launch");
    return VQ2_OK;
}

}  // namespace vq2
