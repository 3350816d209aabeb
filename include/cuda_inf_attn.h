/*
 * cuda_inf_attn.h -- C-ABI of the MI355X (gfx950) attention path of the
 * cuda_inf engine: FP8 E4M3 group-64 KV cache, flash-decoding, fused causal
 * prefill and H2O eviction.
 *
 * Every kernel entry point replaces one __global__ kernel of the reference
 * engine (g023/cuda_inf, src/engine.cu) and keeps its parameter order and
 * pointer roles, so a caller that launched
 *     kernel<<<grid, block>>>(args...)
 * calls
 *     cia_kernel(args..., stream)
 * instead.  The reference's launch site of each kernel is cited beside it.
 *
 * Conventions
 *   - fp16 tensors are passed as uint16_t* (IEEE binary16 bit patterns).
 *   - All pointers are device pointers owned by the caller (hipMalloc'd),
 *     except where "host" is stated.  No entry point allocates device
 *     memory or synchronises: every call is enqueued on `stream`
 *     (a hipStream_t; NULL is the null stream).  Two entry points use a
 *     fixed device array inside the library instead of a workspace
 *     argument (cia_attn_decode_split, cia_attn_decode_noalloc); calls of
 *     them that overlap on one GPU race.  cia_weights_upload
 *     (cuda_inf_model.h) is host I/O and allocates its pinned buffers.
 *   - Every entry point returns CIA_OK (0) or a cia_status code; none calls
 *     exit().  cia_strerror() names the code; after CIA_ERR_HIP,
 *     cia_last_hip_error() returns the hipError_t of the failing call.
 *   - Calls touching the same cache must be serialised by the caller (same
 *     stream, or events), exactly as the reference's single stream does.
 *
 * Shapes are the reference's compile-time constants (engine.cu:22-23, 35-38).
 * Cache layout of one attention layer (engine.cu:596-613, 731-770):
 *     kc8, vc8       uint8  [maxT][CIA_NKV][CIA_HEAD_DIM]   committed FP8
 *     ksc, vsc       fp16   [maxT/64 + 2][CIA_NKV]          group scales
 *     ktail, vtail   fp16   [CIA_KVGROUP][CIA_NKV][CIA_HEAD_DIM]
 *     attn_sum       f32    [maxT]
 *   H2O slot buffer:
 *     kf, vf         uint8  [C][CIA_NKV][CIA_HEAD_DIM]
 *     ks, vs         fp16   [C][CIA_NKV]
 *     slot_pos       int32  [C]           attn_sum  f32 [C]
 *   Flash-decoding partials: pm, pl f32 [CIA_NH*nsplit],
 *     po f32 [CIA_NH*nsplit][CIA_HEAD_DIM], index h*nsplit + split.
 */
#ifndef CUDA_INF_ATTN_H
#define CUDA_INF_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIA_NH 32            /* query heads            (engine.cu:36) */
#define CIA_NKV 8            /* kv heads               (engine.cu:37) */
#define CIA_GQA 4            /* query heads per kv head (engine.cu:38) */
#define CIA_HEAD_DIM 64      /* (engine.cu:35) */
#define CIA_KVGROUP 64       /* tokens per FP8 group   (engine.cu:23) */
#define CIA_E4M3_MAX 448.0f  /* (engine.cu:22) */
#define CIA_HIDDEN 2048       /* hidden size H          (engine.cu:33) */
#define CIA_NSPLIT_DEFAULT 16   /* the reference's NSPLIT (engine.cu:392) */
#define CIA_NSPLIT_MAX 4096

typedef enum cia_status {
  CIA_OK = 0,
  CIA_ERR_NULL = 1,       /* a required pointer is NULL */
  CIA_ERR_ALIGN = 2,      /* a pointer is not aligned as documented */
  CIA_ERR_ARG = 3,        /* an integer argument is out of range */
  CIA_ERR_HIP = 4,        /* a HIP runtime call or launch failed */
  CIA_ERR_STATE = 5,      /* host-side cache state is inconsistent */
  CIA_ERR_NOSLOT = 6,     /* H2O: no slot could be chosen for eviction */
  CIA_ERR_IO = 7          /* a model file could not be opened, read or parsed
                             (include/cuda_inf_model.h) */
} cia_status;

const char* cia_strerror(int status);
int cia_last_hip_error(void);
/* version of this library, e.g. "cuda_inf_attn 0.1 gfx950" */
const char* cia_version(void);

/* ------------------------------------------------------------------ */
/* group-64 FP8 KV cache                                              */
/* ------------------------------------------------------------------ */

/* kv_write_tail (engine.cu:190-198; launch engine.cu:838).
 * Copies cnt fresh tokens k,v [cnt][8][64] into tail rows slot..slot+cnt-1.
 * Requires 0 <= slot, 0 <= cnt, slot + cnt <= 64. */
int cia_kv_write_tail(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                      uint16_t* vtail, int slot, int cnt, void* stream);

/* kv_commit_group (engine.cu:202-228; launch engine.cu:841-842).
 * Per kv head: amax over the 64x64 tail block, scale = amax/448 + 1e-12
 * (fp32), ksc/vsc[grp*8+h] = fp16(scale), FP8 bytes of x/scale into rows
 * dst_tok_base..dst_tok_base+63.  Bytes and scales are bit-exact. */
int cia_kv_commit_group(const uint16_t* ktail, const uint16_t* vtail,
                        uint8_t* kc8, uint8_t* vc8, uint16_t* ksc,
                        uint16_t* vsc, int dst_tok_base, int grp,
                        void* stream);

/* The device E4M3 encoder of f2e4m3 (engine.cu:24-26) that the commit and
 * H2O writers use, exposed for validation: out[i] = e4m3(float bits
 * first_bits + i) for i < n (no kernel counterpart in the reference). */
int cia_e4m3_encode_range(uint32_t first_bits, int64_t n, uint8_t* out,
                          void* stream);

/* ------------------------------------------------------------------ */
/* attention over the group-64 cache                                  */
/* ------------------------------------------------------------------ */

/* attention_fused (engine.cu:236-308; launch engine.cu:854-855).
 * Causal attention for S queries q [S][32][64] at positions past..past+S-1
 * over FP8 keys [0, min(committed, qpos+1)) and tail keys up to qpos.
 * out [S][32][64] fp16.  attn_sum (may be NULL): per-key attention mass is
 * added with the deterministic rule of cia_attention_h2o; it then needs
 * `ws` of ws_bytes >= cia_mass_workspace_bytes(S) bytes (else ws may be NULL
 * and ws_bytes 0); a smaller ws is rejected with CIA_ERR_ARG. */
int cia_attention_fused(const uint16_t* q, const uint8_t* kc8,
                        const uint8_t* vc8, const uint16_t* ksc,
                        const uint16_t* vsc, const uint16_t* ktail,
                        const uint16_t* vtail, int committed, uint16_t* out,
                        float* attn_sum, int S, int past, float scale,
                        void* ws, int64_t ws_bytes, void* stream);

/* EXPERIMENTAL.  The causal attention of attention_fused (engine.cu:236-308)
 * with both products on the OCP-fp8 matrix cores (no counterpart kernel in
 * the reference; same arguments without attn_sum/ws).  K and V are used as
 * the cache's FP8 bytes; Q is quantised to fp8 per (query, head) with scale
 * amax/448 and the softmax numerators per tile, so the output carries that
 * extra rounding: its error against the fp32 reference is reported, it is
 * not held to cia_attention_fused's tolerance.  On MI355X it is slower than
 * cia_attention_fused (141-146 against 100-102 us at 4096 queries: the
 * hi/lo terms that keep its error near fp16's double the contraction, and
 * one fp8 term alone gives 0.09 max errors), so nothing in the library
 * calls it; it is kept to measure the fp8 matrix cores against. */
int cia_attention_fused_fp8(const uint16_t* q, const uint8_t* kc8,
                            const uint8_t* vc8, const uint16_t* ksc,
                            const uint16_t* vsc, const uint16_t* ktail,
                            const uint16_t* vtail, int committed, uint16_t* out,
                            int S, int past, float scale, void* stream);

/* attn_decode_split (engine.cu:396-464; launch engine.cu:848-851).
 * One query (q row 0, [32][64]) at position qpos; keys [0, qpos] are cut
 * into nsplit ranges of ceil((qpos+1)/nsplit) keys, as the reference does
 * per query head.  Writes the partial softmax state (m, l, o) of every
 * (query head, split) to pm/pl/po at index h*nsplit + split.  An empty
 * split writes m = -1e30, l = 0.  nsplit in [1, CIA_NSPLIT_MAX]
 * (the reference fixes 16).  With fewer splits than the launch has
 * workgroups per kv head, each split is shared by several workgroups that
 * meet in a fixed device array inside the library (750 KiB per GPU, held
 * until the process ends): the call allocates nothing and can be captured
 * into a graph, the first call on a device included.  Calls on one GPU
 * share that array, so calls that overlap on one GPU (several streams, or
 * graph replays beside eager calls on another stream) race; such callers
 * use cia_attn_decode_split_ws with a workspace per stream. */
int cia_attn_decode_split(const uint16_t* q, const uint8_t* kc8,
                          const uint8_t* vc8, const uint16_t* ksc,
                          const uint16_t* vsc, const uint16_t* ktail,
                          const uint16_t* vtail, int committed, int qpos,
                          float scale, float* pm, float* pl, float* po,
                          int nsplit, void* stream);

/* attn_decode_split (engine.cu:396-464) with a caller-owned workspace in
 * place of the library's array, for callers that run split decodes on
 * several streams at once: ws of ws_bytes >= cia_split_workspace_bytes(nsplit)
 * bytes, 16-byte aligned, ZEROED before its first use (it holds arrival
 * counters, which every call leaves at zero).  Calls that share a ws must
 * not overlap.  Results are bit-identical to cia_attn_decode_split's. */
int cia_attn_decode_split_ws(const uint16_t* q, const uint8_t* kc8,
                             const uint8_t* vc8, const uint16_t* ksc,
                             const uint16_t* vsc, const uint16_t* ktail,
                             const uint16_t* vtail, int committed, int qpos,
                             float scale, float* pm, float* pl, float* po,
                             int nsplit, void* ws, int64_t ws_bytes,
                             void* stream);
/* workspace bytes of cia_attn_decode_split_ws (0 for nsplit < 1) */
int64_t cia_split_workspace_bytes(int nsplit);

/* attn_decode_combine (engine.cu:467-480; launch engine.cu:852).
 * Merges the nsplit partials of every query head into out [32][64] fp16;
 * splits with l <= 0 are skipped. */
int cia_attn_decode_combine(const float* pm, const float* pl, const float* po,
                            uint16_t* out, int nsplit, void* stream);

/* Flash-decoding with the library's own split on the matrix cores (no
 * counterpart kernel in the reference; it replaces the pair of launches at
 * engine.cu:848-852 and computes the same attention) in ONE launch: up to
 * 32 workgroups per kv head stream the FP8 groups, the first also takes the
 * fp16 tail, and the last workgroup of each kv head to finish merges the
 * partials.  Requires committed <= qpos + 1 (the tail holds keys
 * committed..qpos).  ws: device memory of at least
 * cia_decode_workspace_bytes(qpos + 1) bytes, passed with its size, ZEROED
 * before its first use (it holds per-kv-head arrival counters, which every
 * call leaves at zero again).  Calls that share a ws must not overlap. */
int cia_attn_decode(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                    const uint16_t* ksc, const uint16_t* vsc,
                    const uint16_t* ktail, const uint16_t* vtail,
                    int committed, int qpos, float scale, uint16_t* out,
                    void* ws, int64_t ws_bytes, void* stream);
/* workspace bytes cia_attn_decode needs for contexts of up to max_tokens
 * (also the size of a layer's ws_decode) */
int64_t cia_decode_workspace_bytes(int max_tokens);

/* cia_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a fixed device array inside the library (486 KiB per GPU,
 * held until the process ends; it covers every context); the call allocates
 * nothing.  Calls on one GPU share it: calls that overlap on one GPU
 * (several streams or host threads) race.  Same arguments, results and
 * errors as cia_attn_decode otherwise. */
int cia_attn_decode_noalloc(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                            const uint16_t* ksc, const uint16_t* vsc,
                            const uint16_t* ktail, const uint16_t* vtail,
                            int committed, int qpos, float scale, uint16_t* out,
                            void* stream);

/* A plain streaming read of `bytes` bytes at k and `bytes` at v (one
 * layer's committed FP8 K and V), one launch: the measured memory ceiling
 * the decode kernel is compared against.  No counterpart in the reference
 * (a measurement utility).  bytes: a multiple of 16.  sink: one device
 * uint32, written only on a checksum coincidence. */
int cia_stream_read(const void* k, const void* v, int64_t bytes, uint32_t* sink, void* stream);

/* ------------------------------------------------------------------ */
/* H2O eviction                                                       */
/* ------------------------------------------------------------------ */

/* kv_quant_write (engine.cu:317-333; launch engine.cu:826).
 * Per (token j, kv head h): scale = amax over 64 dims / 448 + 1e-12,
 * FP8 bytes into kf/vf row dst_slots[j] (device int32 [S]),
 * ks/vs[dst_slots[j]*8+h] = fp16(scale).  Bit-exact. */
int cia_kv_quant_write(const uint16_t* k, const uint16_t* v, uint8_t* kf,
                       uint8_t* vf, uint16_t* ks, uint16_t* vs,
                       const int32_t* dst_slots, int S, void* stream);

/* The H2O slot choice of engine.cu:808-825 on the device, followed by
 * kv_quant_write (engine.cu:317-333; launch engine.cu:826): replaces the
 * host loop, its attn_sum fetch, the per-eviction cudaMemset and the
 * dst / slot_pos uploads, so nothing blocks.  Same rule as
 * cia_h2o_pick_slots, same results: token j (position past + j) takes slot
 * *n_live + j while slots are free; after that the slot of least attn_sum
 * (lowest index on ties) among slots with slot_pos <= past + j - W and
 * attn_sum < 1e30, else among all slots with attn_sum < 1e30.  A chosen
 * slot is not chosen again in the call; its attn_sum is cleared to 0 and
 * its slot_pos set to past + j.  slot_pos[C], attn_sum[C] (device) are
 * updated, dst_slots[S] (device) receives each token's slot (-1, and the
 * token is not written, only when every candidate's attn_sum is NaN).
 * When a token takes a slot that an earlier token of the call filled, the
 * slot holds the later token, as after the reference's per-token writes.
 * *n_live (host) advances by the tokens that took free slots.  Returns
 * CIA_ERR_NOSLOT, before any device work, when the call would evict more
 * than C slots.  W >= 0, 0 <= *n_live <= C. */
int cia_h2o_place(const uint16_t* k, const uint16_t* v, uint8_t* kf,
                  uint8_t* vf, uint16_t* ks, uint16_t* vs, float* attn_sum,
                  int32_t* slot_pos, int32_t* dst_slots, int* n_live, int C,
                  int W, int S, int past, void* stream);

/* attention_h2o (engine.cu:337-384; launch engine.cu:827-828).
 * Attention of S queries over the n_live slots whose slot_pos <= qpos;
 * out [S][32][64] fp16.  attn_sum[t] (device f32, required as in the
 * reference) gains the attention mass of every (query, head) with the
 * deterministic rule below, so that the eviction order is reproducible:
 *   s(t) = fma chain over d ascending of q[d]*k(t)[d] from 0, times scale;
 *   per 64-slot block b: m_b = max s, e = expdet(s - m_b), l_b = the
 *   e's xor-butterfly total; m = max m_b, c_b = expdet(m_b - m),
 *   l = sum of l_b * c_b in ascending b; p = e * (c_b * (1/l));
 *   attn_sum[t] += p in (query, head) order.
 * ws: device scratch of ws_bytes >= cia_h2o_workspace_bytes(S, n_live)
 * bytes (16-byte aligned); queries are processed 16 at a time through it. */
int cia_attention_h2o(const uint16_t* q, const uint8_t* kf, const uint8_t* vf,
                      const uint16_t* ks, const uint16_t* vs,
                      const int32_t* slot_pos, int n_live, uint16_t* out,
                      float* attn_sum, int S, int past, float scale, void* ws,
                      int64_t ws_bytes, void* stream);
/* scratch bytes of cia_attention_h2o for S queries over up to C slots */
int64_t cia_h2o_workspace_bytes(int S, int C);
/* scratch bytes of cia_attention_fused's attn_sum option for S queries */
int64_t cia_mass_workspace_bytes(int S);

/* ------------------------------------------------------------------ */
/* QK producers                                                       */
/* ------------------------------------------------------------------ */

/* rmsnorm_head on q, rmsnorm_head on k, then rope (engine.cu:148-182;
 * launches engine.cu:799-801) as one launch, in place on q [S][32][64] and
 * k [S][8][64].  qw, kw: fp16 [64] norm weights; pos: device int32 [S].
 * Fixed-order arithmetic (bit-identical to the CPU restatement): the sum of
 * squares in the reference's tree order, inv = 1/sqrtf(ss/64 + eps),
 * y = fp16((x*inv)*w); RoPE angles pos * theta^(-2d/64) (the exponent table
 * in double, rounded to fp32) with a deterministic sin/cos in place of
 * sinf/cosf; fp16 results after each stage as in the reference. */
int cia_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* qw,
                     const uint16_t* kw, const int32_t* pos, int S, float eps,
                     float theta, void* stream);

/* ------------------------------------------------------------------ */
/* INT4 group-128 projections                                         */
/* ------------------------------------------------------------------ */
/* Weight format of tools/export_weights.py:7-13, 64-79 (the Q4 views of
 * engine.cu:58, 65-71): W [N][K] as packed u8 [N][K/2] (two K-adjacent
 * nibbles per byte, k even in the low nibble) followed by scales fp16
 * [N][K/128]; w[n][k] = (nibble - 8) * scale[n][k/128].  K must be a
 * positive multiple of 128; packed and x 16-byte aligned, scales 2-byte
 * aligned.  Sums are fp32 (order differs from the reference's lanes). */

/* gemv_int4 (engine.cu:83-109) as launched by run_gemv_int4
 * (engine.cu:626-630): y[m][n] = sum_k x[m][k] * w[n][k] for m < M, n < N;
 * x fp16 [M][K], y fp32 [M][N].  M = 0 is a no-op. */
int cia_gemv_int4(const uint16_t* x, const uint8_t* packed,
                  const uint16_t* scales, float* y, int N, int K, int M,
                  void* stream);
/* out_proj and the residual add (engine.cu:858-859, run_gemv_int4 then
 * add_f32_inplace): y[m][n] += sum_k x[m][k] * w[n][k], one launch. */
int cia_gemv_int4_add(const uint16_t* x, const uint8_t* packed,
                      const uint16_t* scales, float* y, int N, int K, int M,
                      void* stream);
/* The q, k and v projections of an attention layer with their fp16
 * conversions (engine.cu:792-797: three run_gemv_int4 and three f32_to_f16)
 * in one launch: q fp16 [M][Nq] = fp16(x Wq^T), k, v fp16 [M][Nkv]; each
 * output is the round-to-nearest-even fp16 of its fp32 sum, as f32_to_f16
 * makes it. */
int cia_qkv_proj_int4(const uint16_t* x, const uint8_t* wq_packed,
                      const uint16_t* wq_scales, int Nq,
                      const uint8_t* wk_packed, const uint16_t* wk_scales,
                      const uint8_t* wv_packed, const uint16_t* wv_scales,
                      int Nkv, int K, int M, uint16_t* q, uint16_t* k,
                      uint16_t* v, void* stream);

/* ------------------------------------------------------------------ */
/* host-side policy (plain C++, no device access)                     */
/* ------------------------------------------------------------------ */

/* One step of the reference's append loop (engine.cu:830-845). */
typedef struct cia_append_op {
  int src_token;    /* first fresh token of this op (offset into k/v) */
  int slot;         /* tail slot it lands in */
  int cnt;          /* tokens copied */
  int commit;       /* 1 if the group fills and is committed after the copy */
  int commit_base;  /* dst_tok_base of that commit (== committed before it) */
  int commit_grp;   /* grp of that commit */
} cia_append_op;

/* Plans the append of S tokens at positions past..past+S-1 given
 * *committed; fills ops[0..*n_ops) (max_ops entries available) and advances
 * *committed.  Requires committed % 64 == 0 and
 * committed <= past <= committed + 64 (the tail holds past-committed
 * tokens).  Returns CIA_ERR_ARG / CIA_ERR_STATE on violations. */
int cia_kv_append_plan(int* committed, int S, int past, cia_append_op* ops,
                       int max_ops, int* n_ops);

/* The reference's H2O clamps (engine.cu:752-756): budget >= prompt,
 * budget <= maxT, window defaults to budget/2, window <= budget-1. */
void cia_h2o_clamp(int* budget, int* window, int prompt_len, int maxT);

/* H2O slot choice for S fresh tokens (engine.cu:808-823), on host arrays:
 * slotpos[C] and *n_live are updated; attn_host[C] is the host copy of the
 * device attention mass (picked slots are overwritten with 1e30 as the
 * reference does).  dst[S] receives the slot of each token, zeroed[S]
 * (may be NULL) 1 where that slot's device attn_sum must be cleared.
 * Returns the number of evictions (>= 0) or -CIA_ERR_NOSLOT. */
int cia_h2o_pick_slots(int* n_live, int C, int W, int32_t* slotpos,
                       float* attn_host, int S, int past, int32_t* dst,
                       int32_t* zeroed);

/* ------------------------------------------------------------------ */
/* layer driver: the attention branch of layer_forward (engine.cu:802-857) */
/* ------------------------------------------------------------------ */

/* Device buffers of one attention layer (caller-owned, engine.cu:596-613)
 * plus the host counters the reference keeps beside them (committed[l],
 * n_live[l]); its host slot positions (slotpos_h[l]) live on the device
 * only, in d_slotpos. */
typedef struct cia_layer {
  /* group-64 cache */
  uint8_t* kc8; uint8_t* vc8; uint16_t* ksc; uint16_t* vsc;
  uint16_t* ktail; uint16_t* vtail;
  int maxT;
  int committed;
  /* flash-decoding */
  int nsplit;            /* 0 -> cia_attn_decode path with ws_decode */
  float* pm; float* pl; float* po;
  void* ws_decode;       /* cia_decode_workspace_bytes(maxT) bytes, zeroed
                            before first use */
  /* H2O (budget > 0 enables it) */
  int budget, window;
  uint8_t* kf; uint8_t* vf; uint16_t* ks; uint16_t* vs;
  float* hattn;          /* device attn_sum [budget] */
  int32_t* d_slotpos;    /* device [budget], slot positions (-1: free) */
  int32_t* d_dst;        /* device [max tokens per call] */
  int n_live;
  void* ws_mass;         /* cia_h2o_workspace_bytes(max tokens per call,
                            budget) bytes */
  /* QK producers (engine.cu:799-801); qw == NULL: q and k arrive prepared.
   * Otherwise q and k are raw and the layer runs per-head RMSNorm (weights
   * qw, kw: fp16 [64], eps) and RoPE (theta) at positions past..past+S-1
   * itself: inside the decode kernels for a single-token step on the
   * group-64 cache, else with one cia_qk_norm_rope launch into prep_ws
   * (device fp16 [prep_cap][40][64], q rows then k rows per token). */
  const uint16_t* qw; const uint16_t* kw;
  float eps, theta;
  uint16_t* prep_ws;
  int prep_cap;
} cia_layer;

/* Append S fresh tokens (k, v: device fp16 [S][8][64]) then attend q
 * (device fp16 [S][32][64]) into out, exactly as engine.cu:799-857 (with
 * the QK producers when L->qw is set; q and k are then only read):
 * H2O when budget > 0, else append + (S == 1 ? flash-decoding : fused).
 * H2O mode chooses slots on the device (cia_h2o_place) where the reference
 * blocks on copies (engine.cu:814, 824-825).  evicted (may be NULL): on
 * return *evicted holds the slot evicted for the last token, or -1; when
 * that token evicted, reading the slot back synchronises `stream`, so pass
 * NULL to keep the call asynchronous. */
int cia_layer_forward(cia_layer* L, const uint16_t* q, const uint16_t* k,
                      const uint16_t* v, uint16_t* out, int S, int past,
                      float scale, int* evicted, void* stream);

/* The placement loop alone (engine.cu:830-845): append S tokens at
 * past..past+S-1 to the group-64 cache, committing every group that fills;
 * no attention.  Used to load a context into the cache. */
int cia_layer_append(cia_layer* L, const uint16_t* k, const uint16_t* v,
                     int S, int past, void* stream);

/* The decode loop of the reference (engine.cu:954-958) restricted to the
 * attention branches: for step s in [0, steps) and layer l in [0, n_layers)
 * runs cia_layer_forward(&layers[l], q[s][l], k[s][l], v[s][l],
 * out[s][l], 1, past + s, ...).  q/out: fp16 [steps][n_layers][32][64],
 * k/v: fp16 [steps][n_layers][8][64].  events (may be NULL): 3*steps*n_layers
 * hipEvent_t; for (step s, layer l), r = s*n_layers + l, events[3r] is
 * recorded before the layer's attention launches (after any separate append
 * launches), events[3r+1] between the first attention launch and the second
 * (after the only one when there is one) and events[3r+2] after the last:
 * per-kernel timing on the stream the kernels run on.  On an H2O layer
 * (budget > 0) events[3r] precedes the slot placement, events[3r+1]
 * follows it and events[3r+2] follows the attention; no evicted slot is
 * read back, so the loop never waits on the stream. */
int cia_decode_loop(cia_layer* layers, int n_layers, const uint16_t* q,
                    const uint16_t* k, const uint16_t* v, uint16_t* out,
                    int past, int steps, float scale, void** events,
                    void* stream);

#define CIA_DECODE_MAX_LAYERS_PER_LAUNCH 8
/* cia_decode_loop with the launch structure chosen: layers_per_launch 1
 * runs every layer's attention in launches of its own (the reference's
 * per-layer structure, engine.cu:846-852); 0 (cia_decode_loop's choice) or
 * 2..8 runs up to that many consecutive layers of a step (at most
 * CIA_DECODE_MAX_LAYERS_PER_LAUNCH) in ONE launch when they qualify: all on
 * the group-64 cache with nsplit 0, the same committed count, the fresh
 * token landing in each tail, the QK producers on all of them or none (one
 * eps and theta), at least 8 committed groups per 64-key range of the
 * launch (about 4096 keys and up), and a grid of one workgroup per compute
 * unit that fits the device.  Otherwise the layer runs alone, as with 1.
 * In one launch layer l + 1's scores start only after every output row of
 * layer l is stored (its q would be computed from them), while its FP8 K/V
 * already stream in; outputs and cache bytes are bit-identical to the
 * per-layer launches.  When all the layers of a step go in one launch and no
 * events are given, consecutive steps run in that same launch too, up to
 * the step whose token fills a group (a run of at most 64 steps): step
 * t + 1's first layer is scored only after step t's last layer has stored
 * its output, as between layers (with the QK producers, each step's RoPE at
 * its own position).  The
 * workspace is the first layer's ws_decode.  With events, every step is a
 * launch of its own, and every layer of such a launch has events[3r]
 * recorded before it and events[3r+1], events[3r+2] after it.  The
 * in-launch wait between layers is bounded: if the grid was not resident
 * at once it gives up and sets the workspace's fault word
 * (cia_decode_fault) rather than hang. */
int cia_decode_loop_ex(cia_layer* layers, int n_layers, const uint16_t* q,
                       const uint16_t* k, const uint16_t* v, uint16_t* out,
                       int past, int steps, float scale,
                       int layers_per_launch, void** events, void* stream);

/* cia_decode_loop_ex with the steps per launch bounded as well:
 * tokens_per_launch 1 launches every step on its own (no runs), n >= 2 at
 * most n steps per run, 0 (cia_decode_loop_ex's choice) runs up to each
 * group fill.  Outputs and cache bytes do not depend on it.  No
 * counterpart in the reference (its decode launches per layer). */
int cia_decode_loop_runs(cia_layer* layers, int n_layers, const uint16_t* q,
                         const uint16_t* k, const uint16_t* v, uint16_t* out,
                         int past, int steps, float scale, int layers_per_launch,
                         int tokens_per_launch, void** events, void* stream);

/* Reads (synchronously) the fault word of a decode workspace: nonzero when a
 * one-launch multi-layer step gave up waiting for a previous layer (its
 * outputs are then not valid).  The word stays set until the workspace is
 * cleared.  No counterpart in the reference. */
int cia_decode_fault(const void* ws, int64_t ws_bytes, int* fault);

/* INT4 projection weights of one attention layer (the Q4 tensors
 * self_attn.{q,k,v,out}_proj.weight of engine.cu:792-797, 858) and the
 * scratch their outputs live in. */
typedef struct cia_attn_proj {
  const uint8_t* q_packed; const uint16_t* q_scales; /* [2048][1024], [2048][16] */
  const uint8_t* k_packed; const uint16_t* k_scales; /* [512][1024],  [512][16]  */
  const uint8_t* v_packed; const uint16_t* v_scales; /* [512][1024],  [512][16]  */
  const uint8_t* o_packed; const uint16_t* o_scales; /* [2048][1024], [2048][16] */
  uint16_t* ws; /* device fp16 scratch of cap * 5120 elements: q, k, v and the
                   attention output of up to cap tokens */
  int cap;
} cia_attn_proj;

/* The attention branch of one layer (engine.cu:792-859): x fp16 [S][2048]
 * (operator_norm's output) -> q, k, v in one launch (cia_qkv_proj_int4),
 * the QK producers (when L->qw is set) and attention through
 * cia_layer_forward, then out_proj added into the residual h fp32
 * [S][2048] in one launch (cia_gemv_int4_add).  S <= P->cap.  A
 * single-token step on a group-64 layer with L->qw set is four launches
 * (projections, attend, finish, out_proj) where the reference makes
 * fourteen. */
int cia_attn_block_forward(cia_layer* L, const cia_attn_proj* P,
                           const uint16_t* x, float* h, int S, int past,
                           float scale, int* evicted, void* stream);

/* Decode steps of the attention branches: for step s and layer l runs
 * cia_attn_block_forward(&layers[l], &proj[l], x[s][l], h, 1, past + s).
 * x: fp16 [steps][n_layers][2048]; h: fp32 [2048], the residual stream
 * every layer adds into.  events (may be NULL): 4*steps*n_layers
 * hipEvent_t; for r = s*n_layers + l, events[4r] precedes the projections,
 * events[4r+1] follows them, events[4r+2] follows the attention and
 * events[4r+3] the out_proj. */
int cia_attn_block_loop(cia_layer* layers, const cia_attn_proj* proj,
                        int n_layers, const uint16_t* x, float* h, int past,
                        int steps, float scale, void** events, void* stream);

#ifdef __cplusplus
}
#endif
#endif
