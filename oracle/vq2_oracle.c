/*
 * vq2_oracle.c -- CPU restatement of the VQ2 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as a checker
 * or as the timed CPU baseline.  The product path (compressai_amd) never
 * links, loads or calls it.
 *
 * Compiled with -O2 -ffp-contract=off so that every float expression rounds
 * exactly as written (no FMA contraction): the dequant is then bit-exact by
 * construction and the fp32-accumulation GEMV follows a fixed, documented
 * summation order.
 *
 * Reference semantics restated here (paths relative to the reference repo):
 *   index decode   vq2/kernels.py:47,72,140,171 (int32(i16) & 0xFFFF),
 *                  vq2/runtime.py:32-35 (_as_index), uint8 stage 2 used as is
 *                  (vq2/kernels.py:48)
 *   unpack_fixed   vq2/export.py:56-70 (16/8/4/12-bit fixed-width packing)
 *   dequant        vq2/vq.py:283-292 (QMat.dequant before rot.inv),
 *                  vq2/benchmark_qualidade_velocidade_35b.py:34-45
 *   VQ GEMV        vq2/kernels.py:32-78 (_vq_gemv_16_8, _vq_gemv_16):
 *                  y[r] = (sum_g sum_j f32(cb[idx][j]) * f32(x[8g+j])) * f32(s[r]) * rs
 *   grouped GEMV   vq2/kernels.py:117-176 (_parallel_moe_gate_up/_down),
 *                  vq2/paged_runtime.py:19-41 (CPU twins)
 *   RHT            vq2/vq.py:22-27,44-87 (hadamard, Rot.fwd/inv):
 *                  fwd(x) = blockdiag_hb(H) (sign .* x[perm]) * scale
 *   top-1          torch.argmax (first maximum), legion/engine.py:288,
 *                  vq2/generate.py:65
 *
 * Parity status of each function is pinned by tests/test_oracle_*.py (see the
 * "pinned by" line in each comment).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>

/* dtype codes, identical to the C-ABI's (include/vq2_amd.h) */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };
/* stage-2 index kinds */
enum { ORC_S2_NONE = 0, ORC_S2_U8 = 1, ORC_S2_U16 = 2 };

/* ---------------------------------------------------------------- scalars */

/* IEEE binary16 -> binary32, exact (normals, subnormals, inf, nan).
 * pinned by: exhaustive comparison with numpy float16->float32. */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24, renormalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* bfloat16 -> binary32, exact.  pinned by: exhaustive vs torch bf16->f32. */
float orc_bf16_to_f32(uint16_t b)
{
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> bfloat16, round to nearest even; NaN kept quiet.
 * pinned by: torch .to(bfloat16) on edge cases + 2^20 random patterns. */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
        return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* binary32 -> binary16, round to nearest even, overflow to inf.
 * pinned by: numpy astype(float16) on edge cases + random patterns. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t au = u & 0x7FFFFFFFu;
    if (au >= 0x7F800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (au > 0x7F800000u ? 0x200u : 0u));
    if (au >= 0x477FF000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (au < 0x38800000u) {
        /* result is subnormal or zero: value / 2^-24 rounded to integer */
        if (au < 0x33000000u) /* < 2^-25: rounds to zero (ties at 2^-25 -> 0) */
            return sign;
        uint32_t e = au >> 23;
        uint32_t m = (au & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14 + (112 - e) ... total shift to 2^-24 units */
        /* value = m * 2^(e-150); in units of 2^-24: m * 2^(e-126) = m >> (126-e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u)))
            q++;
        return (uint16_t)(sign | q);
    }
    /* normal */
    uint32_t e = (au >> 23) - 112u;
    uint32_t m = au & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
        q++;
    return (uint16_t)(sign | q);
}

static inline float ld(const void* p, int dt, int64_t i)
{
    switch (dt) {
    case ORC_F16: return orc_f16_to_f32(((const uint16_t*)p)[i]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

/* --------------------------------------------------------- index decoding */

/* int16 bit pattern -> uint16 code as int32: int32(v) & 0xFFFF.
 * vq2/kernels.py:47, vq2/runtime.py:32-35.
 * pinned by: exhaustive 65536 patterns vs numpy view(uint16). */
void orc_decode_idx16(const int16_t* in, int32_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        out[i] = (int32_t)in[i] & 0xFFFF;
}

/* vq2/export.py:56-70 unpack_fixed for bits in {4, 8, 12, 16}; returns the
 * number of symbols written or -1 on a bad width / short buffer.
 * pinned by: hand-built known-answer packs (tests/test_oracle_decode.py). */
int64_t orc_unpack_fixed(const uint8_t* buf, int64_t nbytes, int bits, int64_t n, int32_t* out)
{
    if (bits == 16) {
        if (nbytes < 2 * n) return -1;
        for (int64_t i = 0; i < n; i++)
            out[i] = (int32_t)buf[2 * i] | ((int32_t)buf[2 * i + 1] << 8);
        return n;
    }
    if (bits == 8) {
        if (nbytes < n) return -1;
        for (int64_t i = 0; i < n; i++) out[i] = buf[i];
        return n;
    }
    if (bits == 4) {
        if (nbytes * 2 < n) return -1;
        for (int64_t i = 0; i < n; i++)
            out[i] = (i & 1) ? (buf[i >> 1] >> 4) : (buf[i >> 1] & 15);
        return n;
    }
    if (bits == 12) {
        if ((n + 1) / 2 * 3 > nbytes) return -1;
        for (int64_t i = 0; i < n; i++) {
            int64_t p = (i >> 1) * 3;
            uint32_t w = (uint32_t)buf[p] | ((uint32_t)buf[p + 1] << 8) | ((uint32_t)buf[p + 2] << 16);
            out[i] = (int32_t)((i & 1) ? (w >> 12) : (w & 4095u));
        }
        return n;
    }
    return -1;
}

static inline int32_t code0(const int16_t* idx0, int64_t i) { return (int32_t)idx0[i] & 0xFFFF; }
static inline int32_t code1(const void* idx1, int kind, int64_t i)
{
    return kind == ORC_S2_U8 ? (int32_t)((const uint8_t*)idx1)[i] : ((int32_t)((const int16_t*)idx1)[i] & 0xFFFF);
}

/* ----------------------------------------------------------------- dequant */

/* Rotated-space weight rows [r0, r1):
 *   W[r, 8g+j] = (f32(cb0[i0][j]) [+ f32(cb1[i1][j])]) * f32(s[r])
 * exactly in that order, each op rounded to fp32 (vq2/vq.py:283-292 with the
 * fp32 codebooks of vq2/benchmark_qualidade_velocidade_35b.py:41-45).
 * out is [(r1-r0), NG*8] fp32.
 * pinned by: bitwise equality with a numpy float32 evaluation and one-hot
 * codebooks (tests/test_oracle_dequant.py). */
void orc_dequant_rows(const int16_t* idx0, const void* idx1, int s2kind,
                      const void* cb0, const void* cb1, int cb_dt,
                      const void* scale, int s_dt,
                      int64_t r0, int64_t r1, int64_t ng, float* out)
{
    for (int64_t r = r0; r < r1; r++) {
        float s = ld(scale, s_dt, r);
        for (int64_t g = 0; g < ng; g++) {
            int64_t i = r * ng + g;
            int32_t a0 = code0(idx0, i);
            int32_t a1 = s2kind ? code1(idx1, s2kind, i) : 0;
            for (int j = 0; j < 8; j++) {
                float w = ld(cb0, cb_dt, (int64_t)a0 * 8 + j);
                if (s2kind) {
                    float w1 = ld(cb1, cb_dt, (int64_t)a1 * 8 + j);
                    w = w + w1;
                }
                out[(r - r0) * ng * 8 + g * 8 + j] = w * s;
            }
        }
    }
}

/* --------------------------------------------------------------- VQ GEMV */

/* Batched VQ GEMV, rows [0, out_rows), batch columns b < batch:
 *   acc = sum_g sum_j (f32(cb0[a0][j]) [+ f32(cb1[a1][j])]) * f32(x[b, 8g+j])
 *   y32[b, r] = (f32(acc32) * f32(s[r])) * rs          (fp32 accumulation)
 *   y64[b, r] = acc64 * s[r] * rs                        (fp64 accumulation)
 * The fp32 accumulation adds each group's 8 products in j order into a group
 * partial, then adds the partial into acc32 (g ascending) -- one fixed order.
 * Either output may be NULL.  x is [batch, x_stride] of dtype x_dt; y is
 * [batch, out_rows].  vq2/kernels.py:32-78 (and the 4 bpw (16,16) variant,
 * which masks stage 2 with & 0xFFFF, vq2/runtime.py:32-35).
 * pinned by: fp64 dense matmul of the dequantized matrix (numpy),
 * one-hot codebooks (y = gathered x entries), linearity in x. */
void orc_vq_gemv(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                 const int16_t* idx0, const void* idx1, int s2kind,
                 const void* cb0, const void* cb1, int cb_dt,
                 const void* scale, int s_dt,
                 int64_t out_rows, int64_t n, float rs,
                 float* y32, double* y64)
{
    int64_t ng = n / 8;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(batch * n));
    for (int64_t b = 0; b < batch; b++)
        for (int64_t k = 0; k < n; k++)
            xf[b * n + k] = ld(x, x_dt, b * x_stride + k);
    float w[8];
    for (int64_t r = 0; r < out_rows; r++) {
        float s = ld(scale, s_dt, r);
        for (int64_t b = 0; b < batch; b++) {
            float acc32 = 0.0f;
            double acc64 = 0.0;
            const float* xb = xf + b * n;
            for (int64_t g = 0; g < ng; g++) {
                int64_t i = r * ng + g;
                int32_t a0 = code0(idx0, i);
                int32_t a1 = s2kind ? code1(idx1, s2kind, i) : 0;
                for (int j = 0; j < 8; j++) {
                    w[j] = ld(cb0, cb_dt, (int64_t)a0 * 8 + j);
                    if (s2kind) w[j] = w[j] + ld(cb1, cb_dt, (int64_t)a1 * 8 + j);
                }
                float part = 0.0f;
                for (int j = 0; j < 8; j++) {
                    float p = w[j] * xb[g * 8 + j];
                    part = part + p;
                    acc64 += (double)w[j] * (double)xb[g * 8 + j];
                }
                acc32 = acc32 + part;
            }
            if (y32) {
                float t = acc32 * s;
                y32[b * out_rows + r] = t * rs;
            }
            if (y64) y64[b * out_rows + r] = acc64 * (double)s * (double)rs;
        }
    }
    free(xf);
}

/* Grouped per-expert VQ GEMV (2 bpw), the semantics of
 * _parallel_moe_gate_up_kernel / _parallel_moe_down_kernel
 * (vq2/kernels.py:117-176) and their CPU twins (vq2/paged_runtime.py:19-41):
 *   e = ids[k];  y[k, r] = (sum cb[pool[e, r, g] & 0xFFFF] . x_k[g]) * s[e, r] * rs
 * x_k = x + k * x_pair_stride (stride 0: one x shared by all pairs, gate_up;
 * stride ng*8: per-pair activations, down).  ids are int32 (ids_i64 == 0) or
 * int64.  An id outside [0, n_experts) yields NaN rows (the product library
 * does the same).
 * pinned by: the dense oracle applied per pair to the expert's slice. */
void orc_moe_grouped(const void* x, int x_dt, int64_t x_pair_stride,
                     const void* ids, int ids_i64, int64_t n_pairs,
                     const int16_t* pool, int64_t n_experts,
                     const void* cb, int cb_dt,
                     const void* pool_scale, int s_dt,
                     int64_t out_rows, int64_t ng, float rs,
                     float* y32, double* y64)
{
    int64_t n = ng * 8;
    for (int64_t k = 0; k < n_pairs; k++) {
        int64_t e = ids_i64 ? ((const int64_t*)ids)[k] : (int64_t)((const int32_t*)ids)[k];
        if (e < 0 || e >= n_experts) {
            for (int64_t r = 0; r < out_rows; r++) {
                if (y32) y32[k * out_rows + r] = NAN;
                if (y64) y64[k * out_rows + r] = NAN;
            }
            continue;
        }
        const int16_t* pe = pool + e * out_rows * ng;
        size_t esz = (s_dt == ORC_F32) ? 4 : 2;
        const char* se = (const char*)pool_scale + (size_t)(e * out_rows) * esz;
        size_t xsz = (x_dt == ORC_F32) ? 4 : 2;
        const char* xk = (const char*)x + (size_t)(k * x_pair_stride) * xsz;
        orc_vq_gemv(xk, x_dt, 1, n, pe, NULL, ORC_S2_NONE, cb, NULL, cb_dt, se, s_dt,
                    out_rows, n, rs, y32 ? y32 + k * out_rows : NULL, y64 ? y64 + k * out_rows : NULL);
    }
}

/* ------------------------------------------------------------------- RHT */

/* In-place unnormalised Walsh-Hadamard transform of v[0..hb) in natural
 * (Sylvester) order: v <- H_hb v with H = [[H, H], [H, -H]]
 * (vq2/vq.py:22-27).  pinned by: scipy.linalg.hadamard dense fp64 matmul. */
static void fwht64(double* v, int64_t hb)
{
    for (int64_t h = 1; h < hb; h <<= 1)
        for (int64_t i = 0; i < hb; i += 2 * h)
            for (int64_t j = i; j < i + h; j++) {
                double a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* Randomised Hadamard transform over the last dim, fp64 internally.
 * forward (inverse == 0), vq2/vq.py:74-76:
 *     v[i] = x[perm[i]] * sign[i];  y_blk = H_hb v_blk * scale
 * inverse (inverse != 0), vq2/vq.py:84-87:
 *     z_blk = H_hb y_blk * scale;  z[i] *= sign[i];  out[perm[i]] = z[i]
 * perm may be NULL (identity), sign may be NULL (all +1).  x and y are
 * [batch, n] fp64.  hb must be a power of two dividing n.
 * Returns 0, or -1 on a bad hb/n. */
int orc_rht(const double* x, double* y, const int32_t* perm, const int8_t* sign,
            int64_t n, int64_t hb, int64_t batch, double scale, int inverse)
{
    if (hb <= 0 || (hb & (hb - 1)) || n % hb) return -1;
    double* v = (double*)malloc(sizeof(double) * (size_t)n);
    for (int64_t b = 0; b < batch; b++) {
        const double* xb = x + b * n;
        double* yb = y + b * n;
        if (!inverse) {
            for (int64_t i = 0; i < n; i++)
                v[i] = xb[perm ? perm[i] : i] * (sign ? (double)sign[i] : 1.0);
            for (int64_t o = 0; o < n; o += hb) fwht64(v + o, hb);
            for (int64_t i = 0; i < n; i++) yb[i] = v[i] * scale;
        } else {
            for (int64_t i = 0; i < n; i++) v[i] = xb[i];
            for (int64_t o = 0; o < n; o += hb) fwht64(v + o, hb);
            for (int64_t i = 0; i < n; i++) {
                double z = v[i] * scale * (sign ? (double)sign[i] : 1.0);
                yb[perm ? perm[i] : i] = z;
            }
        }
    }
    free(v);
    return 0;
}

/* ---------------------------------------------------------------- argmax */

/* First index of the maximum of each row of v [rows, cols] (torch.argmax
 * semantics for NaN-free input).  pinned by: numpy.argmax. */
void orc_argmax_rows(const double* v, int64_t rows, int64_t cols, int64_t* out)
{
    for (int64_t r = 0; r < rows; r++) {
        const double* p = v + r * cols;
        int64_t best = 0;
        for (int64_t c = 1; c < cols; c++)
            if (p[c] > p[best]) best = c;
        out[r] = best;
    }
}

/* ------------------------------------------------------ bulk conversions */
/* Vector forms of the scalar conversions above, for exhaustive pinning. */
void orc_f16_to_f32_n(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}
void orc_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}
void orc_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}
void orc_f32_to_f16_n(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}
