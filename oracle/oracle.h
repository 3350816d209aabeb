/*
 * oracle.h -- scalar CPU restatement of the cuda_inf attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is what the HIP path is compared
 * against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it.  Nothing in cuda_inf_amd/ links or calls it.
 *
 * Every function restates one piece of the reference engine (src/engine.cu of
 * g023/cuda_inf); the citation is given at each declaration.  Shapes are the
 * engine's compile-time constants (engine.cu:22-23, 35-38):
 *   NH = 32 query heads, NKV = 8 kv heads, GQA = 4, D = 64, KVGROUP = 64.
 *
 * Layouts (engine.cu:184-187, 590-613):
 *   q / out        fp16 [S][NH][D]
 *   k / v (fresh)  fp16 [S][NKV][D]
 *   kc8 / vc8      u8   [maxT][NKV][D]      committed FP8 E4M3
 *   ksc / vsc      fp16 [maxT/64+2][NKV]    one scale per (group, kv head)
 *   ktail / vtail  fp16 [KVGROUP][NKV][D]   the in-progress group
 *   pm / pl        f32  [NH*nsplit]         partials, index h*nsplit+sp
 *   po             f32  [NH*nsplit][D]
 *   H2O:  kf/vf u8 [C][NKV][D], ks/vs fp16 [C][NKV], slot_pos i32 [C],
 *         attn_sum f32 [C]
 *
 * fp16 values travel as uint16_t bit patterns.
 *
 * Parity status of each function (how it is pinned) is recorded in the
 * header comment of oracle.c.
 */
#ifndef CUDA_INF_ORACLE_H
#define CUDA_INF_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_NH 32
#define ORC_NKV 8
#define ORC_GQA 4
#define ORC_D 64
#define ORC_KVGROUP 64
#define ORC_E4M3_MAX 448.0f

/* ---- scalar codecs -------------------------------------------------- */
/* IEEE binary16 round-to-nearest-even; the reference's __float2half. */
uint16_t orc_f32_to_f16(float x);
/* exact binary16 -> binary32; the reference's __half2float. */
float orc_f16_to_f32(uint16_t h);
/* OCP OFP8 E4M3, SATFINITE, RNE (engine.cu:24-26 f2e4m3). */
uint8_t orc_e4m3_encode(float x);
/* OCP E4M3 -> fp32, exact (engine.cu:27-30 e4m3f). */
float orc_e4m3_decode(uint8_t b);
/* group scale, amax/448 + 1e-12 in fp32 (engine.cu:218-219, 327). */
float orc_quant_scale(float amax);
/* deterministic exp (Cody-Waite reduction + degree-7 Taylor, explicit fma);
 * the H2O attention-mass definition uses it on both CPU and GPU. */
float orc_exp_det(float x);

/* deterministic sin and cos of an fp32 angle (|x| < 2^20): k = rint(x*2/pi),
 * three-part Cody-Waite reduction with fma, Taylor polynomials (degree 9 /
 * 8, Horner with fma), quadrant by k & 3.  Used by the deterministic RoPE
 * on both CPU and GPU in place of engine.cu:167-168's sinf/cosf. */
void orc_sincos_det(float x, float* s, float* c);
/* RoPE inverse frequencies theta^(-2i/64), i = 0..31, computed in double
 * and rounded to fp32 (engine.cu:166's powf as a table). */
void orc_rope_invf(float theta, float* invf32);
/* Per-head RMSNorm then rotate-half RoPE, in place on q [S][NH][D] and
 * k [S][NKV][D] (engine.cu:148-158 twice, then 161-182, called at
 * 799-801): ss = the reference's tree sum of x^2 (pairs d, d+s for
 * s = 32..1), inv = 1/sqrtf(ss/64 + eps), y = fp16((x*inv)*w); then for
 * d < 32, ang = pos*invf[d], (sn, cs) = sincos_det(ang),
 * y0' = fp16(y0*cs - y1*sn), y1' = fp16(y1*cs + y0*sn), each product and
 * difference rounded separately.  qw, kw: fp16 [64] norm weights. */
void orc_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* qw,
                      const uint16_t* kw, const int32_t* pos, int S, float eps,
                      float theta);

/* bulk helpers (for exhaustive tests through ctypes) */
void orc_f32_to_f16_array(const float* x, uint16_t* out, int64_t n);
void orc_e4m3_encode_array(const float* x, uint8_t* out, int64_t n);
void orc_e4m3_encode_range_u32(uint32_t first_bits, int64_t n, uint8_t* out);
void orc_exp_det_array(const float* x, float* out, int64_t n);
void orc_sincos_det_array(const float* x, float* s, float* c, int64_t n);

/* ---- group-64 KV cache ---------------------------------------------- */
/* engine.cu:190-198 */
void orc_kv_write_tail(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                       uint16_t* vtail, int slot, int cnt);
/* engine.cu:202-228 */
void orc_kv_commit_group(const uint16_t* ktail, const uint16_t* vtail,
                         uint8_t* kc8, uint8_t* vc8, uint16_t* ksc,
                         uint16_t* vsc, int dst_tok_base, int grp);
/* engine.cu:830-845: place S fresh tokens at positions past..past+S-1,
 * committing every group that fills.  *committed is updated in place.
 * Returns the number of groups committed. */
int orc_kv_append(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                  uint16_t* vtail, uint8_t* kc8, uint8_t* vc8, uint16_t* ksc,
                  uint16_t* vsc, int* committed, int S, int past);

/* ---- attention over the group-64 cache ------------------------------ */
/* engine.cu:236-308.  out16 and/or out32 (pre-rounding fp32) may be NULL.
 * attn_sum (may be NULL) is accumulated with the deterministic mass rule
 * documented in oracle.c.  rows: if non-NULL, only the n_rows listed query
 * indices are computed (others untouched). */
void orc_attention_fused(const uint16_t* q, const uint8_t* kc8,
                         const uint8_t* vc8, const uint16_t* ksc,
                         const uint16_t* vsc, const uint16_t* ktail,
                         const uint16_t* vtail, int committed, uint16_t* out16,
                         float* out32, float* attn_sum, int S, int past,
                         float scale, const int* rows, int n_rows);
/* orc_attention_fused's outputs for query heads [h0, h1) of all S rows on
 * nthreads threads (no attn_sum); identical per (row, head) */
void orc_attention_fused_mt(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                            const uint16_t* ksc, const uint16_t* vsc, const uint16_t* ktail,
                            const uint16_t* vtail, int committed, uint16_t* out16, float* out32,
                            int S, int past, float scale, int h0, int h1, int nthreads);

/* engine.cu:396-464 with runtime nsplit (reference: NSPLIT=16) and the
 * reference's 128-thread block structure. */
void orc_attn_decode_split(const uint16_t* q, const uint8_t* kc8,
                           const uint8_t* vc8, const uint16_t* ksc,
                           const uint16_t* vsc, const uint16_t* ktail,
                           const uint16_t* vtail, int committed, int qpos,
                           float scale, float* pm, float* pl, float* po,
                           int nsplit);
/* engine.cu:467-480.  out16 and/or out32 may be NULL. */
void orc_attn_decode_combine(const float* pm, const float* pl, const float* po,
                             uint16_t* out16, float* out32, int nsplit);
/* split + combine, (head, split) units spread over nthreads POSIX threads
 * (the multi-core CPU baseline). */
void orc_attn_decode_mt(const uint16_t* q, const uint8_t* kc8,
                        const uint8_t* vc8, const uint16_t* ksc,
                        const uint16_t* vsc, const uint16_t* ktail,
                        const uint16_t* vtail, int committed, int qpos,
                        float scale, float* pm, float* pl, float* po,
                        int nsplit, uint16_t* out16, float* out32,
                        int nthreads);

/* ---- H2O eviction --------------------------------------------------- */
/* engine.cu:317-333 */
void orc_kv_quant_write(const uint16_t* k, const uint16_t* v, uint8_t* kf,
                        uint8_t* vf, uint16_t* ks, uint16_t* vs,
                        const int32_t* dst_slots, int S);
/* engine.cu:337-384 (outputs) with the deterministic attention-mass rule
 * for attn_sum documented in oracle.c.  out16/out32 may be NULL. */
void orc_attention_h2o(const uint16_t* q, const uint8_t* kf, const uint8_t* vf,
                       const uint16_t* ks, const uint16_t* vs,
                       const int32_t* slot_pos, int n_live, uint16_t* out16,
                       float* out32, float* attn_sum, int S, int past,
                       float scale);
/* engine.cu:808-823 slot choice for S fresh tokens at past..past+S-1.
 * n_live, slotpos[C] are updated in place; attn_sum_host is the host copy of
 * the device attention mass (read; the picked slots are set to 1e30 as the
 * reference does).  dst[S] receives the slots; zeroed[S] (may be NULL)
 * receives 1 where the device attn_sum of dst[j] must be cleared.  Returns the
 * number of evictions. */
int orc_h2o_pick_slots(int* n_live, int C, int W, int32_t* slotpos,
                       float* attn_sum_host, int S, int past, int32_t* dst,
                       int32_t* zeroed);

/* ---- INT4 group-128 projections ------------------------------------ */
/* The weight format of tools/export_weights.py:7-13, 64-79: W fp32 [N][K]
 * (K a multiple of 128) -> packed u8 [N][K/2] (k even in the low nibble,
 * nibble = q + 8) and scales fp16 [N][K/128].  Per group: amax = max |w|,
 * scale = amax / 7 (fp32 division), q = round-half-even(w / scale') with
 * scale' = scale or 1 when scale is 0, clipped to [-7, 7]; the stored
 * scale is fp16(scale). */
void orc_quant_int4_g128(const float* w, int N, int K, uint8_t* packed,
                         uint16_t* scales);
/* engine.cu:83-109 (gemv_int4, launched per row block by run_gemv_int4,
 * 626-630): y[m][n] = sum_k x[m][k] * (nib(n,k) - 8) * scale[n][k/128],
 * x fp16 [M][K], y fp32 [M][N].  The reference sums in fp32 in its lane
 * order; this restatement sums the exact products in fp64 (the value the
 * reference's sum approximates) and rounds once.  absum (may be NULL)
 * receives sum_k |x * w| in fp64 rounded to fp32, the scale of the
 * summation error. */
void orc_gemv_int4(const uint16_t* x, const uint8_t* packed,
                   const uint16_t* scales, float* y, float* absum, int N, int K,
                   int M);

#ifdef __cplusplus
}
#endif
#endif
