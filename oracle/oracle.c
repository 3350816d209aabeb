/*
 * oracle.c -- scalar CPU restatement of the cuda_inf attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY (what the HIP path is compared against, never
 * the thing measured or shipped).  Loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, nowhere else.
 *
 * Reference: g023/cuda_inf src/engine.cu (cited as engine.cu:LINE).  The
 * reference's own build needs nvcc and cuda_fp8.h, neither of which exists in
 * this image, so it cannot be compiled as a second oracle; this file is the
 * only restatement.
 *
 * How each function is pinned (the tests live in tests/test_oracle_*.py):
 *   orc_f32_to_f16        exhaustive over all 2^32 inputs against numpy's
 *                         float32->float16 cast (an independent RNE).
 *   orc_e4m3_encode       OCP OFP8 E4M3 definition: every decision threshold
 *                         (midpoints between neighbouring codes, and one ulp
 *                         either side), ties-to-even, +-0, SATFINITE at and
 *                         beyond 448 and infinity, NaN; plus brute-force
 *                         nearest-code search on random inputs.
 *   orc_e4m3_decode       closed-form table of all 256 codes.
 *   orc_quant_scale       closed forms (amax 0 -> 1e-12 -> fp16 0; amax 448).
 *   orc_exp_det           relative error against double exp over a dense
 *                         sweep, and exp(0) == 1 exactly.
 *   kv_write_tail/commit  integer invariants and closed-form groups
 *                         (zero group, single non-zero element -> 0x7E,
 *                         constant group).
 *   kv_append             committed count and tail contents for arbitrary
 *                         batch sequences against a direct simulation.
 *   attention_fused       brute-force fp64 softmax attention on the
 *                         dequantised cache; invariants (all-equal V, one
 *                         key, q = 0 gives the mean of V).
 *   attn_decode_split/
 *   combine               equal to the last row of attention_fused within
 *                         fp32 rounding; nsplit in {1,16,256,512} agree;
 *                         empty splits skipped; fp64 brute force.
 *   kv_quant_write        closed-form per-token cases as for commit.
 *   attention_h2o         fp64 brute force for the output; the attention
 *                         mass against an fp64 restatement, and one-hot
 *                         constructions that force known masses.
 *   h2o_pick_slots        hand-checked cases: lowest-slot tie break, the
 *                         window rule pos <= posj - W, the fallback scan.
 *   sincos_det            error against float64 sin/cos (<= 2e-7 up to
 *                         2.6e5), exact values at 0, odd/even symmetry bit
 *                         for bit, sin^2 + cos^2 = 1.
 *   rope_invf             float32 rounding of float64 theta^(-2i/64).
 *   quant_int4_g128       closed forms: a group of amax 7 (scale 1) with
 *                         ties at +-0.5, 1.5, 2.5 (half-to-even), a zero
 *                         group (scale 0, nibbles 8), one non-zero element
 *                         placed at even / odd k and in each group (nibble
 *                         order, group index); |w - dequant| <= scale/2 and
 *                         the amax element at nibble 1 or 15 on random
 *                         weights.
 *   gemv_int4             an independent numpy fp64 product of the
 *                         dequantised dense matrix; one-hot x gives a
 *                         dequantised column exactly; constant nibbles give
 *                         scale * sum(x).
 *   qk_norm_rope          an independent numpy float32 restatement of the
 *                         norm (tree-ordered sum of squares) and rotation;
 *                         unit-RMS rows, pair norms kept, position 0 is the
 *                         identity; within one fp16 step of the torch
 *                         producers (fp32 torch cos/sin).
 *
 * Deterministic attention mass (used where the reference accumulates
 * attn_sum with atomicAdd, engine.cu:291-307, 371-383).  The reference's sum
 * order is undefined and its __expf is approximate, so the evicted-slot
 * sequence it produces is not reproducible even on its own GPU.  Both this
 * oracle and the HIP kernels therefore compute the mass with the following
 * rule, which is bit-reproducible on any IEEE-754 machine:
 *   for query i (qpos = past+i) and query head h (kv head h/4):
 *     kd(t)[d] = e4m3(byte) * scale   (exact in fp32)  or the fp16 tail value
 *     s(t)     = fmaf-chain over d = 0..63 of q[d]*kd(t)[d], from 0.0f,
 *                then times `scale` (the 1/sqrt(64) softmax scale)
 *     (the slots in blocks b of 64: slot t = 64b + j, j = 0..63)
 *     m_b      = max of s(t) over the eligible t of block b (-inf if none)
 *     m        = max of m_b over the blocks
 *     e(t)     = exp_det(s(t) - m_b) for eligible t, else 0
 *     l_b      = the block's 64 values v[j] = e(64b + j) (0 past the end)
 *                reduced by six butterfly steps v[j] = v[j] + v[j ^ off]
 *                for off = 32,16,8,4,2,1; l_b = v[0]
 *     c_b      = exp_det(m_b - m), 0 for a block with no eligible slot
 *     l        = l_b * c_b added in ascending b from 0.0f
 *     w_b      = c_b * (1.0f / l)
 *     p(t)     = e(t) * w_b
 *   attn_sum[t] += p(t), one add per (i, h) in ascending i then ascending h.
 * The sum order is one of the orders the reference's atomics can produce.
 *
 * fp16 <-> fp32, E4M3 and all arithmetic on the bit-exact paths use IEEE
 * binary32 with round-to-nearest-even; the file is compiled with
 * -ffp-contract=off so that every fused multiply-add is an explicit fmaf.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define NH ORC_NH
#define NKV ORC_NKV
#define GQA ORC_GQA
#define D ORC_D
#define G ORC_KVGROUP

/* hot loops get an FMA-instruction clone, chosen at load time */
#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define ORC_HOT __attribute__((target_clones("fma", "default")))
#else
#define ORC_HOT
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* IEEE binary16, round to nearest even                               */
/* ------------------------------------------------------------------ */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) {
    if (ax == 0x7F800000u) return sign | 0x7C00u;
    return sign | 0x7E00u | (uint16_t)((ax >> 13) & 0x3FFu); /* quiet NaN */
  }
  if (ax >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520 rounds to inf */
  if (ax >= 0x38800000u) {                      /* fp16 normal range */
    uint32_t h = ((((ax >> 23) - 112u)) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | (uint16_t)h;
  }
  if (ax <= 0x33000000u) return sign; /* <= 2^-25: ties to the even zero */
  {
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e; /* units of 2^-24 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return sign | (uint16_t)h;
  }
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
  if (e != 0) return u2f(sign | ((e + 112u) << 23) | (m << 13));
  if (m == 0) return u2f(sign);
  /* subnormal: m * 2^-24, exact in fp32 */
  {
    float v = (float)m * 5.9604644775390625e-08f;
    return (sign ? -v : v);
  }
}

/* ------------------------------------------------------------------ */
/* OCP OFP8 E4M3: bias 7, max 448 = S.1111.110, NaN = S.1111.111,     */
/* no infinities, subnormal step 2^-9.  SATFINITE: |x| >= 448 and     */
/* +-inf encode to +-448; NaN keeps its sign (S.1111.111).            */
/* ------------------------------------------------------------------ */
uint8_t orc_e4m3_encode(float f) {
  uint32_t x = f2u(f);
  uint8_t sign = (uint8_t)((x >> 24) & 0x80u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return sign | 0x7Fu;  /* NaN */
  if (ax >= 0x43E00000u) return sign | 0x7Eu; /* >= 448 (and inf): saturate */
  if (ax >= 0x3C800000u) {                    /* >= 2^-6: normal code */
    uint32_t h = (((ax >> 23) - 120u) << 3) | ((ax & 0x7FFFFFu) >> 20);
    uint32_t rem = ax & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (h & 1u))) h++;
    if (h > 0x7Eu) h = 0x7Eu;
    return sign | (uint8_t)h;
  }
  if (ax <= 0x3A800000u) return sign; /* <= 2^-10: ties to the even zero */
  {
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 141u - e; /* units of 2^-9 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return sign | (uint8_t)h; /* h == 8 is the smallest normal, 0x08 */
  }
}

static float e4m3_closed_form(uint8_t b) {
  uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 0xFu && m == 7u) v = NAN;
  else if (e == 0) v = (float)m * 0.001953125f; /* m * 2^-9 */
  else v = ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  return (b & 0x80u) ? -v : v;
}

static float g_e4m3_table[256];
__attribute__((constructor)) static void init_e4m3_table(void) {
  for (int b = 0; b < 256; b++) g_e4m3_table[b] = e4m3_closed_form((uint8_t)b);
}

float orc_e4m3_decode(uint8_t b) { return g_e4m3_table[b]; }

float orc_quant_scale(float amax) {
  return amax / ORC_E4M3_MAX + 1e-12f; /* IEEE division, then the add */
}

/* ------------------------------------------------------------------ */
/* deterministic exp: Cody-Waite two-constant reduction by ln2, then  */
/* a degree-7 Taylor polynomial in Horner form with explicit fmaf,    */
/* then an exact power-of-two scale.  Inputs below -60 return 0 (the  */
/* result and anything derived from it then stay clear of fp32        */
/* subnormals, whose handling differs between machines).              */
/* ------------------------------------------------------------------ */
ORC_HOT float orc_exp_det(float x) {
  if (!(x >= -60.0f)) return (x != x) ? x : 0.0f;
  if (x > 88.0f) return INFINITY;
  float kf = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-kf, 0.693145751953125f, x);
  r = fmaf(-kf, 1.428606765330187045e-06f, r);
  float p = 1.98412701138295233249664306640625e-04f; /* 1/5040 */
  p = fmaf(p, r, 1.38888892810791730880737304687500e-03f); /* 1/720 */
  p = fmaf(p, r, 8.33333376795053482055664062500000e-03f); /* 1/120 */
  p = fmaf(p, r, 4.16666679084300994873046875000000e-02f); /* 1/24 */
  p = fmaf(p, r, 1.66666671633720397949218750000000e-01f); /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int k = (int)kf;
  return p * u2f((uint32_t)(k + 127) << 23);
}

static inline float h2f_(uint16_t h) { return orc_f16_to_f32(h); }

/* ------------------------------------------------------------------ */
/* deterministic sin / cos and the QK producers                       */
/* ------------------------------------------------------------------ */
void orc_sincos_det(float x, float* s, float* c) {
  const float kf = rintf(x * 0x1.45f306p-1f);    /* x * 2/pi */
  float r = fmaf(-kf, 0x1.921fb6p+0f, x);         /* pi/2 in three parts */
  r = fmaf(-kf, -0x1.777a5cp-25f, r);
  r = fmaf(-kf, -0x1.ee59dap-50f, r);
  const float r2 = r * r;
  float ps = fmaf(r2, 0x1.71de3ap-19f, -0x1.a01a02p-13f); /* 1/9!, -1/7! */
  ps = fmaf(r2, ps, 0x1.111112p-7f);                      /* 1/5! */
  ps = fmaf(r2, ps, -0x1.555556p-3f);                     /* -1/3! */
  const float sr = fmaf(r * r2, ps, r);
  float pc = fmaf(r2, 0x1.a01a02p-16f, -0x1.6c16c2p-10f); /* 1/8!, -1/6! */
  pc = fmaf(r2, pc, 0x1.555556p-5f);                      /* 1/4! */
  pc = fmaf(r2, pc, -0x1p-1f);                            /* -1/2 */
  const float cr = fmaf(r2, pc, 1.0f);
  switch (((int)kf) & 3) {
    case 0: *s = sr; *c = cr; break;
    case 1: *s = cr; *c = -sr; break;
    case 2: *s = -sr; *c = -cr; break;
    default: *s = -cr; *c = sr; break;
  }
}

void orc_rope_invf(float theta, float* invf32) {
  for (int i = 0; i < D / 2; i++) invf32[i] = (float)pow((double)theta, -(2.0 * i) / D);
}

/* one head row in place: RMSNorm (tree order of engine.cu:153-154) then RoPE */
static void qk_row(uint16_t* row, const uint16_t* w, int32_t pos, float eps, const float* invf) {
  float v[D], y[D];
  for (int d = 0; d < D; d++) {
    const float x = h2f_(row[d]);
    v[d] = x * x;
  }
  for (int st = D / 2; st > 0; st >>= 1)
    for (int d = 0; d < st; d++) v[d] = v[d] + v[d + st];
  const float inv = 1.0f / sqrtf(v[0] / (float)D + eps);
  for (int d = 0; d < D; d++) y[d] = h2f_(orc_f32_to_f16((h2f_(row[d]) * inv) * h2f_(w[d])));
  for (int d = 0; d < D / 2; d++) {
    float sn, cs;
    orc_sincos_det((float)pos * invf[d], &sn, &cs);
    const float x0 = y[d], x1 = y[d + D / 2];
    row[d] = orc_f32_to_f16(x0 * cs - x1 * sn);
    row[d + D / 2] = orc_f32_to_f16(x1 * cs + x0 * sn);
  }
}

void orc_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* qw, const uint16_t* kw,
                      const int32_t* pos, int S, float eps, float theta) {
  float invf[D / 2];
  orc_rope_invf(theta, invf);
  for (int i = 0; i < S; i++) {
    for (int h = 0; h < NH; h++) qk_row(q + ((size_t)i * NH + h) * D, qw, pos[i], eps, invf);
    for (int h = 0; h < NKV; h++) qk_row(k + ((size_t)i * NKV + h) * D, kw, pos[i], eps, invf);
  }
}

void orc_sincos_det_array(const float* x, float* s, float* c, int64_t n) {
  for (int64_t i = 0; i < n; i++) orc_sincos_det(x[i], &s[i], &c[i]);
}

void orc_f32_to_f16_array(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}
void orc_e4m3_encode_array(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_e4m3_encode(x[i]);
}
void orc_e4m3_encode_range_u32(uint32_t first_bits, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; i++)
    out[i] = orc_e4m3_encode(u2f(first_bits + (uint32_t)i));
}
void orc_exp_det_array(const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_exp_det(x[i]);
}

static inline float h2f(uint16_t h) { return orc_f16_to_f32(h); }

/* ------------------------------------------------------------------ */
/* group-64 KV cache                                                  */
/* ------------------------------------------------------------------ */
/* engine.cu:190-198: tail rows slot..slot+cnt-1 <- k/v rows 0..cnt-1 */
void orc_kv_write_tail(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                       uint16_t* vtail, int slot, int cnt) {
  size_t n = (size_t)cnt * NKV * D, dst = (size_t)slot * NKV * D;
  memcpy(ktail + dst, k, n * 2);
  memcpy(vtail + dst, v, n * 2);
}

/* engine.cu:202-228: per kv head, absmax over the 64x64 block (K and V
 * separately), fp32 scale amax/448+1e-12, stored as fp16, bytes encoded
 * with the fp32 scale. */
void orc_kv_commit_group(const uint16_t* ktail, const uint16_t* vtail,
                         uint8_t* kc8, uint8_t* vc8, uint16_t* ksc,
                         uint16_t* vsc, int dst_tok_base, int grp) {
  for (int h = 0; h < NKV; h++) {
    float mk = 0.f, mv = 0.f;
    for (int t = 0; t < G; t++)
      for (int d = 0; d < D; d++) {
        size_t off = ((size_t)t * NKV + h) * D + d;
        mk = fmaxf(mk, fabsf(h2f(ktail[off])));
        mv = fmaxf(mv, fabsf(h2f(vtail[off])));
      }
    float sck = orc_quant_scale(mk), scv = orc_quant_scale(mv);
    ksc[grp * NKV + h] = orc_f32_to_f16(sck);
    vsc[grp * NKV + h] = orc_f32_to_f16(scv);
    for (int t = 0; t < G; t++)
      for (int d = 0; d < D; d++) {
        size_t off = ((size_t)t * NKV + h) * D + d;
        size_t dst = ((size_t)(dst_tok_base + t) * NKV + h) * D + d;
        kc8[dst] = orc_e4m3_encode(h2f(ktail[off]) / sck);
        vc8[dst] = orc_e4m3_encode(h2f(vtail[off]) / scv);
      }
  }
}

/* engine.cu:830-845 */
int orc_kv_append(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                  uint16_t* vtail, uint8_t* kc8, uint8_t* vc8, uint16_t* ksc,
                  uint16_t* vsc, int* committed, int S, int past) {
  int placed = 0, ncommit = 0;
  while (placed < S) {
    int gpos = past + placed;
    int slot = gpos - *committed;
    int can = S - placed < G - slot ? S - placed : G - slot;
    orc_kv_write_tail(k + (size_t)placed * NKV * D, v + (size_t)placed * NKV * D,
                      ktail, vtail, slot, can);
    placed += can;
    if (slot + can == G) {
      orc_kv_commit_group(ktail, vtail, kc8, vc8, ksc, vsc, *committed,
                          *committed / G);
      *committed += G;
      ncommit++;
    }
  }
  return ncommit;
}

/* ------------------------------------------------------------------ */
/* shared pieces of the attention restatements                        */
/* ------------------------------------------------------------------ */
/* the dequantised key/value row t of kv head kvh in the group-64 cache:
 * FP8 with its group scale for t < committed, the fp16 tail otherwise. */
static void row_group64(const uint8_t* c8, const uint16_t* sc,
                        const uint16_t* tail, int committed, int t, int kvh,
                        float* out) {
  if (t < committed) {
    float s = h2f(sc[(t / G) * NKV + kvh]);
    const uint8_t* p = c8 + ((size_t)t * NKV + kvh) * D;
    for (int d = 0; d < D; d++) out[d] = orc_e4m3_decode(p[d]) * s;
  } else {
    const uint16_t* p = tail + ((size_t)(t - committed) * NKV + kvh) * D;
    for (int d = 0; d < D; d++) out[d] = h2f(p[d]);
  }
}

/* s_raw = fmaf chain over d ascending of q[d]*k[d] starting at 0.0f */
static inline float dot_chain(const float* q, const float* k) {
  float acc = 0.0f;
  for (int d = 0; d < D; d++) acc = fmaf(q[d], k[d], acc);
  return acc;
}

/* chains for n keys at once, keys stored transposed kT[d][n]; same
 * arithmetic as dot_chain per key, vectorisable across keys. */
ORC_HOT static void dot_chain_many(const float* q, const float* kT, int n,
                                   float* out) {
  for (int t = 0; t < n; t++) out[t] = 0.0f;
  for (int d = 0; d < D; d++) {
    const float qd = q[d];
    const float* kr = kT + (size_t)d * n;
    for (int t = 0; t < n; t++) out[t] = fmaf(qd, kr[t], out[t]);
  }
}

/* the mass rule: given the scaled scores s[0..n) and an eligibility mask,
 * write p[0..n) (file header: block maxima m_b, numerators against them,
 * block totals by butterfly, weighted by exp_det(m_b - m) in block order). */
ORC_HOT static void mass_from_scores(const float* s, const unsigned char* ok,
                                     int n, float* e_scratch, float* p) {
  const int nb = (n + 63) / 64;
  float* mb = (float*)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
  float* wb = (float*)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
  float m = -INFINITY;
  for (int b = 0; b < nb; b++) {
    float x = -INFINITY;
    for (int t = 64 * b; t < n && t < 64 * b + 64; t++)
      if (ok[t] && s[t] > x) x = s[t];
    for (int t = 64 * b; t < n && t < 64 * b + 64; t++)
      e_scratch[t] = ok[t] ? orc_exp_det(s[t] - x) : 0.0f;
    if (x > m) m = x;
    mb[b] = x;
  }
  float l = 0.0f;
  for (int b = 0; b < nb; b++) {
    float v[64];
    for (int j = 0; j < 64; j++) v[j] = 64 * b + j < n ? e_scratch[64 * b + j] : 0.0f;
    for (int off = 32; off >= 1; off >>= 1) {
      float w[64];
      for (int j = 0; j < 64; j++) w[j] = v[j] + v[j ^ off];
      memcpy(v, w, sizeof v);
    }
    const float cb = mb[b] == -INFINITY ? 0.0f : orc_exp_det(mb[b] - m);
    wb[b] = cb;
    l = l + v[0] * cb;
  }
  const float inv = 1.0f / l;
  for (int b = 0; b < nb; b++) wb[b] = wb[b] * inv;
  for (int t = 0; t < n; t++) p[t] = e_scratch[t] * wb[t / 64];
  free(mb);
  free(wb);
}

/* ------------------------------------------------------------------ */
/* attention_fused, engine.cu:236-308                                 */
/* ------------------------------------------------------------------ */
/* one (query i, head h) of attention_fused over the dequantised cache */
static void fused_row_head(const uint16_t* q, const float* kd, const float* vd, int i, int h,
                           int past, float scale, uint16_t* out16, float* out32, float* s) {
  int qpos = past + i;
  int kvh = h / GQA;
  float qreg[D];
  for (int d = 0; d < D; d++) qreg[d] = h2f(q[((size_t)i * NH + h) * D + d]);
  /* one online-softmax pass in key order, fp32 (engine.cu:255-285) */
  float m = -1e30f, l = 0.f, o[D];
  for (int d = 0; d < D; d++) o[d] = 0.f;
  for (int t = 0; t <= qpos; t++) {
    const float* kr = kd + ((size_t)t * NKV + kvh) * D;
    const float* vr = vd + ((size_t)t * NKV + kvh) * D;
    float st = dot_chain(qreg, kr) * scale;
    if (s) s[t] = st;
    float mnew = fmaxf(m, st), c = expf(m - mnew), pe = expf(st - mnew);
    l = fmaf(l, c, pe);
    for (int d = 0; d < D; d++) o[d] = fmaf(pe, vr[d], o[d] * c);
    m = mnew;
  }
  float inv = 1.f / l;
  for (int d = 0; d < D; d++) {
    float r = o[d] * inv;
    size_t oi = ((size_t)i * NH + h) * D + d;
    if (out32) out32[oi] = r;
    if (out16) out16[oi] = orc_f32_to_f16(r);
  }
}

/* the cache's keys 0..T-1 dequantised, [t][kv head][d] */
static void dequant_cache(const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
                          const uint16_t* vsc, const uint16_t* ktail, const uint16_t* vtail,
                          int committed, int T, float* kd, float* vd) {
  for (int t = 0; t < T; t++)
    for (int h = 0; h < NKV; h++) {
      row_group64(kc8, ksc, ktail, committed, t, h, kd + ((size_t)t * NKV + h) * D);
      row_group64(vc8, vsc, vtail, committed, t, h, vd + ((size_t)t * NKV + h) * D);
    }
}

void orc_attention_fused(const uint16_t* q, const uint8_t* kc8,
                         const uint8_t* vc8, const uint16_t* ksc,
                         const uint16_t* vsc, const uint16_t* ktail,
                         const uint16_t* vtail, int committed, uint16_t* out16,
                         float* out32, float* attn_sum, int S, int past,
                         float scale, const int* rows, int n_rows) {
  int nq = rows ? n_rows : S;
  int T = past + S; /* keys 0..T-1 exist */
  float* kd = (float*)malloc(sizeof(float) * (size_t)T * NKV * D);
  float* vd = (float*)malloc(sizeof(float) * (size_t)T * NKV * D);
  dequant_cache(kc8, vc8, ksc, vsc, ktail, vtail, committed, T, kd, vd);
  float* s = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
  float* e = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
  float* p = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
  unsigned char* ok = (unsigned char*)malloc((size_t)(T > 0 ? T : 1));
  for (int qi = 0; qi < nq; qi++) {
    int i = rows ? rows[qi] : qi;
    int qpos = past + i;
    for (int h = 0; h < NH; h++) {
      fused_row_head(q, kd, vd, i, h, past, scale, out16, out32, s);
      if (attn_sum) {
        for (int t = 0; t <= qpos; t++) ok[t] = 1;
        mass_from_scores(s, ok, qpos + 1, e, p);
        for (int t = 0; t <= qpos; t++) attn_sum[t] = attn_sum[t] + p[t];
      }
    }
  }
  free(kd); free(vd); free(s); free(e); free(p); free(ok);
}

/* attention_fused's outputs (no attn_sum) for query heads [h0, h1) of every
 * row, rows dealt round-robin to nthreads threads; each (row, head) is the
 * same computation as orc_attention_fused's, so the results are identical */
struct fused_job {
  const uint16_t* q;
  const float* kd;
  const float* vd;
  uint16_t* out16;
  float* out32;
  int S, past, h0, h1, nthreads, tix;
  float scale;
};

static void* fused_worker(void* arg) {
  struct fused_job* j = (struct fused_job*)arg;
  for (int i = j->tix; i < j->S; i += j->nthreads)
    for (int h = j->h0; h < j->h1; h++)
      fused_row_head(j->q, j->kd, j->vd, i, h, j->past, j->scale, j->out16, j->out32, NULL);
  return NULL;
}

void orc_attention_fused_mt(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                            const uint16_t* ksc, const uint16_t* vsc, const uint16_t* ktail,
                            const uint16_t* vtail, int committed, uint16_t* out16, float* out32,
                            int S, int past, float scale, int h0, int h1, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  if (h0 < 0) h0 = 0;
  if (h1 > NH) h1 = NH;
  int T = past + S;
  float* kd = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * NKV * D);
  float* vd = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * NKV * D);
  dequant_cache(kc8, vc8, ksc, vsc, ktail, vtail, committed, T, kd, vd);
  pthread_t th[256];
  struct fused_job jobs[256];
  for (int i = 0; i < nthreads; i++) {
    struct fused_job jb = {q, kd, vd, out16, out32, S, past, h0, h1, nthreads, i, scale};
    jobs[i] = jb;
  }
  for (int i = 1; i < nthreads; i++) pthread_create(&th[i], NULL, fused_worker, &jobs[i]);
  fused_worker(&jobs[0]);
  for (int i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
  free(kd); free(vd);
}

/* ------------------------------------------------------------------ */
/* flash-decoding, engine.cu:396-480                                  */
/* ------------------------------------------------------------------ */
#define ADEC_THREADS 128

static void decode_unit(const uint16_t* q, const uint8_t* kc8,
                        const uint8_t* vc8, const uint16_t* ksc,
                        const uint16_t* vsc, const uint16_t* ktail,
                        const uint16_t* vtail, int committed, int qpos,
                        float scale, float* pm, float* pl, float* po,
                        int nsplit, int h, int sp) {
  int kvh = h / GQA;
  float qs[D];
  for (int d = 0; d < D; d++) qs[d] = h2f(q[(size_t)h * D + d]);
  int total = qpos + 1;
  int chunk = (total + nsplit - 1) / nsplit;
  int kstart = sp * chunk;
  int kend = total < kstart + chunk ? total : kstart + chunk;
  /* per-thread online softmax (engine.cu:417-444) */
  static __thread float tm[ADEC_THREADS], tl[ADEC_THREADS];
  static __thread float to[ADEC_THREADS][D];
  for (int tid = 0; tid < ADEC_THREADS; tid++) {
    float m = -1e30f, l = 0.f, o[D], kr[D], vr[D];
    for (int d = 0; d < D; d++) o[d] = 0.f;
    for (int t = kstart + tid; t < kend; t += ADEC_THREADS) {
      row_group64(kc8, ksc, ktail, committed, t, kvh, kr);
      row_group64(vc8, vsc, vtail, committed, t, kvh, vr);
      float s = dot_chain(qs, kr) * scale;
      float mnew = fmaxf(m, s), c = expf(m - mnew), p = expf(s - mnew);
      l = fmaf(l, c, p);
      for (int d = 0; d < D; d++) o[d] = fmaf(p, vr[d], o[d] * c);
      m = mnew;
    }
    tm[tid] = m; tl[tid] = l;
    memcpy(to[tid], o, sizeof o);
  }
  /* block reduction (engine.cu:446-461): max, then rescale, then a
   * shared-memory tree with strides 64, 32, ..., 1 */
  float bm = -1e30f;
  {
    float red[ADEC_THREADS];
    memcpy(red, tm, sizeof red);
    for (int s = ADEC_THREADS >> 1; s > 0; s >>= 1)
      for (int tid = 0; tid < s; tid++) red[tid] = fmaxf(red[tid], red[tid + s]);
    bm = red[0];
  }
  for (int tid = 0; tid < ADEC_THREADS; tid++) {
    float alpha = expf(tm[tid] - bm);
    tl[tid] = tl[tid] * alpha;
    for (int d = 0; d < D; d++) to[tid][d] = to[tid][d] * alpha;
  }
  for (int s = ADEC_THREADS >> 1; s > 0; s >>= 1)
    for (int tid = 0; tid < s; tid++) {
      tl[tid] += tl[tid + s];
      for (int d = 0; d < D; d++) to[tid][d] += to[tid + s][d];
    }
  int pi = h * nsplit + sp;
  pm[pi] = bm;
  pl[pi] = tl[0];
  for (int d = 0; d < D; d++) po[(size_t)pi * D + d] = to[0][d];
}

void orc_attn_decode_split(const uint16_t* q, const uint8_t* kc8,
                           const uint8_t* vc8, const uint16_t* ksc,
                           const uint16_t* vsc, const uint16_t* ktail,
                           const uint16_t* vtail, int committed, int qpos,
                           float scale, float* pm, float* pl, float* po,
                           int nsplit) {
  for (int h = 0; h < NH; h++)
    for (int sp = 0; sp < nsplit; sp++)
      decode_unit(q, kc8, vc8, ksc, vsc, ktail, vtail, committed, qpos, scale,
                  pm, pl, po, nsplit, h, sp);
}

void orc_attn_decode_combine(const float* pm, const float* pl, const float* po,
                             uint16_t* out16, float* out32, int nsplit) {
  for (int h = 0; h < NH; h++)
    for (int d = 0; d < D; d++) {
      float gm = -1e30f;
      for (int s = 0; s < nsplit; s++) gm = fmaxf(gm, pm[h * nsplit + s]);
      float l = 0.f, acc = 0.f;
      for (int s = 0; s < nsplit; s++) {
        int pi = h * nsplit + s;
        if (pl[pi] <= 0.f) continue;
        float w = expf(pm[pi] - gm);
        l = fmaf(pl[pi], w, l);
        acc = fmaf(po[(size_t)pi * D + d], w, acc);
      }
      float r = acc / l;
      if (out32) out32[h * D + d] = r;
      if (out16) out16[h * D + d] = orc_f32_to_f16(r);
    }
}

struct mt_job {
  const uint16_t *q, *ktail, *vtail, *ksc, *vsc;
  const uint8_t *kc8, *vc8;
  int committed, qpos, nsplit, nthreads, tix;
  float scale, *pm, *pl, *po;
};

static void* mt_worker(void* arg) {
  struct mt_job* j = (struct mt_job*)arg;
  int units = NH * j->nsplit;
  for (int u = j->tix; u < units; u += j->nthreads)
    decode_unit(j->q, j->kc8, j->vc8, j->ksc, j->vsc, j->ktail, j->vtail,
                j->committed, j->qpos, j->scale, j->pm, j->pl, j->po,
                j->nsplit, u / j->nsplit, u % j->nsplit);
  return NULL;
}

void orc_attn_decode_mt(const uint16_t* q, const uint8_t* kc8,
                        const uint8_t* vc8, const uint16_t* ksc,
                        const uint16_t* vsc, const uint16_t* ktail,
                        const uint16_t* vtail, int committed, int qpos,
                        float scale, float* pm, float* pl, float* po,
                        int nsplit, uint16_t* out16, float* out32,
                        int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  struct mt_job jobs[256];
  for (int i = 0; i < nthreads; i++) {
    struct mt_job j = {q, ktail, vtail, ksc, vsc, kc8, vc8, committed, qpos,
                       nsplit, nthreads, i, scale, pm, pl, po};
    jobs[i] = j;
  }
  for (int i = 1; i < nthreads; i++) pthread_create(&th[i], NULL, mt_worker, &jobs[i]);
  mt_worker(&jobs[0]);
  for (int i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
  orc_attn_decode_combine(pm, pl, po, out16, out32, nsplit);
}

/* ------------------------------------------------------------------ */
/* H2O, engine.cu:317-384, 808-823                                    */
/* ------------------------------------------------------------------ */
void orc_kv_quant_write(const uint16_t* k, const uint16_t* v, uint8_t* kf,
                        uint8_t* vf, uint16_t* ks, uint16_t* vs,
                        const int32_t* dst_slots, int S) {
  for (int j = 0; j < S; j++)
    for (int h = 0; h < NKV; h++) {
      const uint16_t* kr = k + ((size_t)j * NKV + h) * D;
      const uint16_t* vr = v + ((size_t)j * NKV + h) * D;
      float mk = 0.f, mv = 0.f;
      for (int d = 0; d < D; d++) {
        mk = fmaxf(mk, fabsf(h2f(kr[d])));
        mv = fmaxf(mv, fabsf(h2f(vr[d])));
      }
      float sck = orc_quant_scale(mk), scv = orc_quant_scale(mv);
      int slot = dst_slots[j];
      size_t dst = ((size_t)slot * NKV + h) * D;
      for (int d = 0; d < D; d++) {
        kf[dst + d] = orc_e4m3_encode(h2f(kr[d]) / sck);
        vf[dst + d] = orc_e4m3_encode(h2f(vr[d]) / scv);
      }
      ks[slot * NKV + h] = orc_f32_to_f16(sck);
      vs[slot * NKV + h] = orc_f32_to_f16(scv);
    }
}

void orc_attention_h2o(const uint16_t* q, const uint8_t* kf, const uint8_t* vf,
                       const uint16_t* ks, const uint16_t* vs,
                       const int32_t* slot_pos, int n_live, uint16_t* out16,
                       float* out32, float* attn_sum, int S, int past,
                       float scale) {
  int n = n_live > 0 ? n_live : 1;
  /* dequantised K transposed per kv head [kvh][d][t], V as [t][kvh][d] */
  float* kT = (float*)malloc(sizeof(float) * (size_t)NKV * D * n);
  float* vd = (float*)malloc(sizeof(float) * (size_t)n * NKV * D);
  for (int t = 0; t < n_live; t++)
    for (int h = 0; h < NKV; h++) {
      float sk = h2f(ks[t * NKV + h]), sv = h2f(vs[t * NKV + h]);
      const uint8_t* kp = kf + ((size_t)t * NKV + h) * D;
      const uint8_t* vp = vf + ((size_t)t * NKV + h) * D;
      for (int d = 0; d < D; d++) {
        kT[((size_t)h * D + d) * n + t] = orc_e4m3_decode(kp[d]) * sk;
        vd[((size_t)t * NKV + h) * D + d] = orc_e4m3_decode(vp[d]) * sv;
      }
    }
  float* s = (float*)malloc(sizeof(float) * n);
  float* e = (float*)malloc(sizeof(float) * n);
  float* p = (float*)malloc(sizeof(float) * n);
  unsigned char* ok = (unsigned char*)malloc(n);
  for (int i = 0; i < S; i++) {
    int qpos = past + i;
    for (int t = 0; t < n_live; t++) ok[t] = slot_pos[t] <= qpos;
    for (int h = 0; h < NH; h++) {
      int kvh = h / GQA;
      float qreg[D];
      for (int d = 0; d < D; d++) qreg[d] = h2f(q[((size_t)i * NH + h) * D + d]);
      dot_chain_many(qreg, kT + (size_t)kvh * D * n, n_live, s);
      for (int t = 0; t < n_live; t++) s[t] = s[t] * scale;
      if (out16 || out32) {
        /* the reference's online softmax in slot order (engine.cu:353-370) */
        float m = -1e30f, l = 0.f, o[D];
        for (int d = 0; d < D; d++) o[d] = 0.f;
        for (int t = 0; t < n_live; t++) {
          if (!ok[t]) continue;
          const float* vr = vd + ((size_t)t * NKV + kvh) * D;
          float mnew = fmaxf(m, s[t]), c = expf(m - mnew), pe = expf(s[t] - mnew);
          l = fmaf(l, c, pe);
          for (int d = 0; d < D; d++) o[d] = fmaf(pe, vr[d], o[d] * c);
          m = mnew;
        }
        float inv = 1.f / l;
        for (int d = 0; d < D; d++) {
          float r = o[d] * inv;
          size_t oi = ((size_t)i * NH + h) * D + d;
          if (out32) out32[oi] = r;
          if (out16) out16[oi] = orc_f32_to_f16(r);
        }
      }
      if (attn_sum) {
        mass_from_scores(s, ok, n_live, e, p);
        for (int t = 0; t < n_live; t++)
          if (ok[t]) attn_sum[t] = attn_sum[t] + p[t];
      }
    }
  }
  free(kT); free(vd); free(s); free(e); free(p); free(ok);
}

/* engine.cu:808-823 */
int orc_h2o_pick_slots(int* n_live, int C, int W, int32_t* slotpos,
                       float* attn_sum_host, int S, int past, int32_t* dst,
                       int32_t* zeroed) {
  int evictions = 0;
  for (int j = 0; j < S; j++) {
    int posj = past + j, slot;
    if (zeroed) zeroed[j] = 0;
    if (*n_live < C) {
      slot = (*n_live)++;
    } else {
      int best = -1;
      float bv = 1e30f;
      for (int t = 0; t < C; t++)
        if (slotpos[t] <= posj - W && attn_sum_host[t] < bv) { bv = attn_sum_host[t]; best = t; }
      if (best < 0)
        for (int t = 0; t < C; t++)
          if (attn_sum_host[t] < bv) { bv = attn_sum_host[t]; best = t; }
      if (best < 0) return -1; /* nothing below 1e30: the reference would index -1 */
      slot = best;
      attn_sum_host[slot] = 1e30f;
      if (zeroed) zeroed[j] = 1;
      evictions++;
    }
    slotpos[slot] = posj;
    dst[j] = slot;
  }
  return evictions;
}

/* tools/export_weights.py:64-79 */
void orc_quant_int4_g128(const float* w, int N, int K, uint8_t* packed, uint16_t* scales) {
  const int ng = K / 128;
  for (int n = 0; n < N; n++)
    for (int g = 0; g < ng; g++) {
      const float* wg = w + (size_t)n * K + (size_t)g * 128;
      float amax = 0.0f;
      for (int i = 0; i < 128; i++) {
        const float a = fabsf(wg[i]);
        if (a > amax) amax = a;
      }
      const float scale = amax / 7.0f;
      const float safe = scale == 0.0f ? 1.0f : scale;
      scales[(size_t)n * ng + g] = orc_f32_to_f16(scale);
      uint8_t* pr = packed + (size_t)n * (K / 2) + (size_t)g * 64;
      for (int i = 0; i < 128; i += 2) {
        int nib[2];
        for (int e = 0; e < 2; e++) {
          float qv = rintf(wg[i + e] / safe); /* ties to even */
          if (qv < -7.0f) qv = -7.0f;
          if (qv > 7.0f) qv = 7.0f;
          nib[e] = (int)qv + 8;
        }
        pr[i / 2] = (uint8_t)(nib[0] | (nib[1] << 4));
      }
    }
}

/* engine.cu:83-109 */
void orc_gemv_int4(const uint16_t* x, const uint8_t* packed, const uint16_t* scales, float* y,
                   float* absum, int N, int K, int M) {
  const int ng = K / 128;
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      const uint8_t* pr = packed + (size_t)n * (K / 2);
      const uint16_t* sr = scales + (size_t)n * ng;
      const uint16_t* xr = x + (size_t)m * K;
      double acc = 0.0, aab = 0.0;
      for (int k = 0; k < K; k++) {
        const uint8_t b = pr[k >> 1];
        const int nib = (k & 1) ? (b >> 4) : (b & 0xF);
        const double wv = (double)(nib - 8) * (double)orc_f16_to_f32(sr[k >> 7]);
        const double t = (double)orc_f16_to_f32(xr[k]) * wv;
        acc += t;
        aab += fabs(t);
      }
      y[(size_t)m * N + n] = (float)acc;
      if (absum) absum[(size_t)m * N + n] = (float)aab;
    }
}
