// host.hip -- host side of the cuda_inf attention path: status codes, the
// append planner (engine.cu:830-845), the H2O clamps and slot picker
// (engine.cu:752-756, 808-823) and the attention branch of layer_forward
// (engine.cu:802-857) driving the gfx950 kernels through the C-ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "cuda_inf_attn.h"

extern "C" __attribute__((visibility("hidden"))) int cia_kv_append_batched(
    const uint16_t* k, const uint16_t* v, uint16_t* ktail, uint16_t* vtail, uint8_t* kc8,
    uint8_t* vc8, uint16_t* ksc, uint16_t* vsc, int* committed, int S, int past, int maxT,
    void* stream);

extern "C" __attribute__((visibility("hidden"))) int cia_decode_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, uint16_t* ktail, uint16_t* vtail, const uint16_t* knew,
    const uint16_t* vnew, int committed, int qpos, float scale, uint16_t* out, void* ws,
    int64_t ws_bytes, void* stream, void* mid_event, const void* prep);

extern "C" __attribute__((visibility("hidden"))) int cia_h2o_decode_step(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
    uint16_t* ks, uint16_t* vs, float* attn_sum, int32_t* slot_pos, int32_t* dst_slots,
    int* n_live, int C, int W, int past, uint16_t* out, float scale, void* ws, int64_t ws_bytes,
    void* stream, void* mid_event, int keys_valid);

extern "C" __attribute__((visibility("hidden"))) int cia_qk_prep_into(
    const uint16_t* q, const uint16_t* k, const uint16_t* qw, const uint16_t* kw, uint16_t* oq,
    uint16_t* ok, int pos0, int S, float eps, float theta, void* stream);

extern "C" __attribute__((visibility("hidden"))) int cia_decode_tok_fits(const cia_layer* L,
                                                                          int nl, int past);

extern "C" __attribute__((visibility("hidden"))) int cia_decode_tok(
    const cia_layer* L, int nl, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    uint16_t* out, int past, float scale, int ntok, int64_t qs, int64_t kvs, void* stream);

extern "C" __attribute__((visibility("hidden"))) const void* cia_qk_prep_desc(
    const uint16_t* qw, const uint16_t* kw, float eps, float theta);

namespace cia {

static thread_local int g_last_hip = 0;

void set_hip_error(hipError_t e) { g_last_hip = (int)e; }

int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  return CIA_OK;
}

static int hip_check(hipError_t e) {
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  return CIA_OK;
}

}  // namespace cia

using namespace cia;

extern "C" const char* cia_strerror(int status) {
  switch (status) {
    case CIA_OK: return "ok";
    case CIA_ERR_NULL: return "required pointer is NULL";
    case CIA_ERR_ALIGN: return "pointer is not aligned as required";
    case CIA_ERR_ARG: return "integer argument out of range";
    case CIA_ERR_HIP: return "HIP runtime call or kernel launch failed";
    case CIA_ERR_STATE: return "cache state inconsistent (tail would exceed 64 tokens)";
    case CIA_ERR_NOSLOT: return "H2O: no slot below 1e30 could be evicted";
    case CIA_ERR_IO: return "model file could not be opened, read or parsed";
    default: return "unknown status";
  }
}

extern "C" int cia_last_hip_error(void) { return g_last_hip; }

extern "C" const char* cia_version(void) { return "cuda_inf_attn 0.1 gfx950"; }

// ---------------------------------------------------------------- append plan
extern "C" int cia_kv_append_plan(int* committed, int S, int past, cia_append_op* ops,
                                  int max_ops, int* n_ops) {
  if (!committed || !n_ops || (!ops && S > 0)) return CIA_ERR_NULL;
  if (S < 0 || past < 0 || *committed < 0 || *committed % CIA_KVGROUP) return CIA_ERR_ARG;
  // the tail holds tokens committed..past-1, so past - committed in [0, 64)
  if (past < *committed || past - *committed >= CIA_KVGROUP) return CIA_ERR_STATE;
  int placed = 0, n = 0, c = *committed;
  while (placed < S) {
    const int gpos = past + placed;
    const int slot = gpos - c;
    const int can = std::min(S - placed, CIA_KVGROUP - slot);
    if (n >= max_ops) return CIA_ERR_ARG;
    cia_append_op& op = ops[n++];
    op.src_token = placed;
    op.slot = slot;
    op.cnt = can;
    placed += can;
    op.commit = (slot + can == CIA_KVGROUP);
    op.commit_base = c;
    op.commit_grp = c / CIA_KVGROUP;
    if (op.commit) c += CIA_KVGROUP;
  }
  *committed = c;
  *n_ops = n;
  return CIA_OK;
}

// ---------------------------------------------------------------- H2O policy
extern "C" void cia_h2o_clamp(int* budget, int* window, int prompt_len, int maxT) {
  if (*budget < prompt_len) *budget = prompt_len;
  if (*budget > maxT) *budget = maxT;
  if (*window <= 0) *window = *budget / 2;
  if (*window >= *budget) *window = *budget - 1;
}

extern "C" int cia_h2o_pick_slots(int* n_live, int C, int W, int32_t* slotpos, float* attn_host,
                                  int S, int past, int32_t* dst, int32_t* zeroed) {
  int evictions = 0;
  for (int j = 0; j < S; j++) {
    const int posj = past + j;
    int slot;
    if (zeroed) zeroed[j] = 0;
    if (*n_live < C) {
      slot = (*n_live)++;
    } else {
      int best = -1;
      float bv = 1e30f;
      for (int t = 0; t < C; t++)  // outside the window, strict <: lowest slot wins ties
        if (slotpos[t] <= posj - W && attn_host[t] < bv) {
          bv = attn_host[t];
          best = t;
        }
      if (best < 0)
        for (int t = 0; t < C; t++)
          if (attn_host[t] < bv) {
            bv = attn_host[t];
            best = t;
          }
      if (best < 0) return -CIA_ERR_NOSLOT;
      slot = best;
      attn_host[slot] = 1e30f;  // never pick the same slot twice in one batch
      if (zeroed) zeroed[j] = 1;
      evictions++;
    }
    slotpos[slot] = posj;
    dst[j] = slot;
  }
  return evictions;
}

// ---------------------------------------------------------------- layer driver
namespace {

// A layer with QK producers (qw set) must have them complete
int prep_check(const cia_layer* L) {
  if (!L->qw) return CIA_OK;
  if (!L->kw) return CIA_ERR_NULL;
  if (!(L->eps >= 0.0f) || !(L->theta > 0.0f) || L->theta == __builtin_inff()) return CIA_ERR_ARG;
  return CIA_OK;
}

// engine.cu:799-801 for the unfused paths: the producers run into the
// layer's prep_ws and q / k then point at the prepared rows
int prep_qk(cia_layer* L, const uint16_t*& q, const uint16_t*& k, int S, int past,
            void* stream) {
  if (!L->qw) return CIA_OK;
  if (!L->prep_ws) return CIA_ERR_NULL;
  if (S > L->prep_cap) return CIA_ERR_ARG;
  uint16_t* oq = L->prep_ws;
  uint16_t* ok = L->prep_ws + (size_t)L->prep_cap * CIA_NH * CIA_HEAD_DIM;
  const int st = cia_qk_prep_into(q, k, L->qw, L->kw, oq, ok, past, S, L->eps, L->theta, stream);
  if (st) return st;
  q = oq;
  k = ok;
  return CIA_OK;
}

// the decode kernels' descriptor when they run the producers themselves
const void* layer_prep(const cia_layer* L) {
  return L->qw ? cia_qk_prep_desc(L->qw, L->kw, L->eps, L->theta) : nullptr;
}

// engine.cu:803-828 with the slot choice on the device: place + quantise,
// then attention with the mass update; no host round trip
// keys_valid: the previous call on L was a single-token step at past - 1
// (within one cia_decode_loop call), whose mass launch left this step's
// placement keys in L->ws_mass
int h2o_forward(cia_layer* L, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                uint16_t* out, int S, int past, float scale, int* evicted, void* stream,
                void* mid_event = nullptr, bool keys_valid = false) {
  const int C = L->budget;
  if (!L->kf || !L->vf || !L->ks || !L->vs || !L->hattn || !L->d_slotpos || !L->d_dst ||
      !L->ws_mass)
    return CIA_ERR_NULL;
  const int n0 = L->n_live;
  int st = prep_qk(L, q, k, S, past, stream);
  if (st) return st;
  if (S == 1) {
    // one token: placed and quantised inside the attention's first launch
    st = cia_h2o_decode_step(q, k, v, L->kf, L->vf, L->ks, L->vs, L->hattn, L->d_slotpos,
                             L->d_dst, &L->n_live, C, L->window, past, out, scale, L->ws_mass,
                             cia_h2o_workspace_bytes(1, C), stream, mid_event, keys_valid);
    if (st) return st;
  } else {
    st = cia_h2o_place(k, v, L->kf, L->vf, L->ks, L->vs, L->hattn, L->d_slotpos, L->d_dst,
                       &L->n_live, C, L->window, S, past, stream);
    if (st) return st;
    if (mid_event && (st = hip_check(hipEventRecord((hipEvent_t)mid_event, (hipStream_t)stream))))
      return st;
    st = cia_attention_h2o(q, L->kf, L->vf, L->ks, L->vs, L->d_slotpos, L->n_live, out,
                           L->hattn, S, past, scale, L->ws_mass, cia_h2o_workspace_bytes(S, C),
                           stream);
    if (st) return st;
  }
  // the last token evicted iff it found no free slot
  if (evicted && n0 + S > C) {
    int32_t slot = -1;
    st = hip_check(hipMemcpyAsync(&slot, L->d_dst + (S - 1), sizeof(slot), hipMemcpyDeviceToHost,
                                  (hipStream_t)stream));
    if (st) return st;
    if ((st = hip_check(hipStreamSynchronize((hipStream_t)stream)))) return st;
    *evicted = slot;
  }
  return CIA_OK;
}

// placement loop (engine.cu:830-845): copy into the tail, commit full
// groups -- one launch for all the groups the tokens complete and one for
// the tail (the reference: one copy and one commit launch per group)
int group64_append(cia_layer* L, const uint16_t* k, const uint16_t* v, int S, int past,
                   void* stream) {
  if (past + S > L->maxT) return CIA_ERR_ARG;
  int committed = L->committed;
  const int st = cia_kv_append_batched(k, v, L->ktail, L->vtail, L->kc8, L->vc8, L->ksc, L->vsc,
                                       &committed, S, past, L->maxT, stream);
  if (st) return st;
  L->committed = committed;
  return CIA_OK;
}

int group64_attend(cia_layer* L, const uint16_t* q, uint16_t* out, int S, int past, float scale,
                   void* stream, void* mid_event = nullptr) {
  if (S == 1) {
    if (L->nsplit > 0) {
      int st = cia_attn_decode_split(q, L->kc8, L->vc8, L->ksc, L->vsc, L->ktail, L->vtail,
                                     L->committed, past, scale, L->pm, L->pl, L->po, L->nsplit,
                                     stream);
      if (st) return st;
      if (mid_event && (st = hip_check(hipEventRecord((hipEvent_t)mid_event, (hipStream_t)stream))))
        return st;
      return cia_attn_decode_combine(L->pm, L->pl, L->po, out, L->nsplit, stream);
    }
    if (L->committed > past + 1 || past - L->committed >= CIA_KVGROUP) return CIA_ERR_STATE;
    return cia_decode_mfma(q, L->kc8, L->vc8, L->ksc, L->vsc, L->ktail, L->vtail, nullptr,
                           nullptr, L->committed, past, scale, out, L->ws_decode,
                           cia_decode_workspace_bytes(L->maxT), stream, mid_event, nullptr);
  }
  int st = cia_attention_fused(q, L->kc8, L->vc8, L->ksc, L->vsc, L->ktail, L->vtail,
                               L->committed, out, nullptr, S, past, scale, nullptr, 0, stream);
  if (st) return st;
  if (mid_event) return hip_check(hipEventRecord((hipEvent_t)mid_event, (hipStream_t)stream));
  return CIA_OK;
}

// Single-token decode on the matrix cores with the append fused in: the
// fresh token's tail write, and the group commit when it completes the
// group, ride in the attention launches (no kv_write_tail / kv_commit_group
// launches).  Usable when the token lands in the current tail.
bool fused_append_ok(const cia_layer* L, int past) {
  const int slot = past - L->committed;
  return L->nsplit == 0 && slot >= 0 && slot < CIA_KVGROUP && past < L->maxT &&
         (slot < CIA_KVGROUP - 1 || L->committed + CIA_KVGROUP <= L->maxT);
}

int decode_fused_append(cia_layer* L, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        uint16_t* out, int past, float scale, void* stream,
                        void* mid_event = nullptr) {
  // q and k arrive raw on a layer with producers: the decode kernels run them
  const int st = cia_decode_mfma(q, L->kc8, L->vc8, L->ksc, L->vsc, L->ktail, L->vtail, k, v,
                                 L->committed, past, scale, out, L->ws_decode,
                                 cia_decode_workspace_bytes(L->maxT), stream, mid_event,
                                 layer_prep(L));
  if (st == CIA_OK && past - L->committed == CIA_KVGROUP - 1) L->committed += CIA_KVGROUP;
  return st;
}

}  // namespace

extern "C" int cia_layer_forward(cia_layer* L, const uint16_t* q, const uint16_t* k,
                                 const uint16_t* v, uint16_t* out, int S, int past, float scale,
                                 int* evicted, void* stream) {
  if (!L || !q || !k || !v || !out) return CIA_ERR_NULL;
  if (S < 1 || past < 0) return CIA_ERR_ARG;
  if (evicted) *evicted = -1;
  int st = prep_check(L);
  if (st) return st;
  if (L->budget > 0) return h2o_forward(L, q, k, v, out, S, past, scale, evicted, stream);
  if (S == 1 && fused_append_ok(L, past))
    return decode_fused_append(L, q, k, v, out, past, scale, stream);
  if ((st = prep_qk(L, q, k, S, past, stream))) return st;
  st = group64_append(L, k, v, S, past, stream);
  if (st) return st;
  return group64_attend(L, q, out, S, past, scale, stream);
}

extern "C" int cia_layer_append(cia_layer* L, const uint16_t* k, const uint16_t* v, int S,
                                int past, void* stream) {
  if (!L || !k || !v) return CIA_ERR_NULL;
  if (S < 0 || past < 0) return CIA_ERR_ARG;
  if (L->budget > 0) return CIA_ERR_STATE;  // H2O layers place tokens by policy
  if (L->qw) return CIA_ERR_STATE;  // raw k needs its q: use cia_layer_forward
  return S ? group64_append(L, k, v, S, past, stream) : CIA_OK;
}

// Steps pos, pos + 1, .. (at most max_steps) that one k_decode_tok launch
// can run: the layers qualify at pos, and the run stops at the step whose
// token fills the group and at every layer's capacity.  0: none.
static int decode_run(const cia_layer* layers, int n_layers, int pos, int max_steps) {
  if (max_steps < 2 || !cia_decode_tok_fits(layers, n_layers, pos)) return 0;
  const int c = layers[0].committed;  // (the same in every layer: fits)
  int run = std::min(max_steps, CIA_KVGROUP - (pos - c));
  for (int j = 0; j < n_layers; j++) run = std::min(run, layers[j].maxT - pos);
  if (pos + run - 1 - c == CIA_KVGROUP - 1) {
    bool fits = true;
    for (int j = 0; j < n_layers; j++) fits = fits && c + CIA_KVGROUP <= layers[j].maxT;
    if (!fits) run--;  // (the commit would not fit: the run stops before it)
  }
  return run;
}

extern "C" int cia_decode_loop_runs(cia_layer* layers, int n_layers, const uint16_t* q,
                                    const uint16_t* k, const uint16_t* v, uint16_t* out,
                                    int past, int steps, float scale, int layers_per_launch,
                                    int tokens_per_launch, void** events, void* stream) {
  if (!layers || !q || !k || !v || !out) return CIA_ERR_NULL;
  if (n_layers < 1 || steps < 0 || past < 0 || layers_per_launch < 0 || tokens_per_launch < 0)
    return CIA_ERR_ARG;
  const int tok_max = tokens_per_launch == 0 ? CIA_KVGROUP : std::min(tokens_per_launch, CIA_KVGROUP);
  for (int l = 0; l < n_layers; l++) {
    const int st = prep_check(&layers[l]);
    if (st) return st;
  }
  const int per = layers_per_launch == 0 ? CIA_DECODE_MAX_LAYERS_PER_LAUNCH
                                         : std::min(layers_per_launch, CIA_DECODE_MAX_LAYERS_PER_LAUNCH);
  const size_t qrow = (size_t)CIA_NH * CIA_HEAD_DIM, krow = (size_t)CIA_NKV * CIA_HEAD_DIM;
  hipStream_t s = (hipStream_t)stream;
  for (int i = 0; i < steps; i++) {
    const int pos = past + i;
    // A run of steps (at most tok_max) in one launch when every layer of a
    // step goes in one launch and no per-step events are asked for: the
    // steps up to the one that fills the group (it ends the run; the next
    // run's FP8 groups include it).
    if (!events && per > 1 && n_layers <= per && tok_max > 1) {
      const int run = decode_run(layers, n_layers, pos, std::min(steps - i, tok_max));
      if (run > 1) {
        const size_t r = (size_t)i * n_layers;
        const int st = cia_decode_tok(layers, n_layers, q + r * qrow, k + r * krow, v + r * krow,
                                      out + r * qrow, pos, scale, run, (int64_t)n_layers * qrow,
                                      (int64_t)n_layers * krow, stream);
        if (st) return st;
        const int last = pos + run - 1;
        for (int j = 0; j < n_layers; j++)
          if (last - layers[j].committed == CIA_KVGROUP - 1) layers[j].committed += CIA_KVGROUP;
        i += run - 1;
        continue;
      }
    }
    for (int l = 0; l < n_layers;) {
      const size_t r = (size_t)i * n_layers + l;
      int st;
      // the next layers of this step in one launch, when they qualify
      const int chunk = std::min(per, n_layers - l);
      if (per > 1 && cia_decode_tok_fits(&layers[l], chunk, pos)) {
        if (events)
          for (int j = 0; j < chunk; j++)
            if ((st = hip_check(hipEventRecord((hipEvent_t)events[3 * (r + j)], s)))) return st;
        st = cia_decode_tok(&layers[l], chunk, q + r * qrow, k + r * krow, v + r * krow,
                            out + r * qrow, pos, scale, 1, 0, 0, stream);
        if (st) return st;
        if (events)
          for (int j = 0; j < chunk; j++)
            for (int e = 1; e < 3; e++)
              if ((st = hip_check(hipEventRecord((hipEvent_t)events[3 * (r + j) + e], s)))) return st;
        for (int j = 0; j < chunk; j++) {
          cia_layer* Lj = &layers[l + j];
          if (pos - Lj->committed == CIA_KVGROUP - 1) Lj->committed += CIA_KVGROUP;
        }
        l += chunk;
        continue;
      }
      cia_layer* L = &layers[l];
      if (L->budget > 0) {
        if (events && (st = hip_check(hipEventRecord((hipEvent_t)events[3 * r], s)))) return st;
        st = h2o_forward(L, q + r * qrow, k + r * krow, v + r * krow, out + r * qrow, 1, pos,
                         scale, nullptr, stream, events ? events[3 * r + 1] : nullptr, i > 0);
        if (st) return st;
        if (events && (st = hip_check(hipEventRecord((hipEvent_t)events[3 * r + 2], s)))) return st;
        l++;
        continue;
      }
      const bool fused = fused_append_ok(L, pos);
      const uint16_t* qi = q + r * qrow;
      const uint16_t* ki = k + r * krow;
      if (!fused) {
        if ((st = prep_qk(L, qi, ki, 1, pos, stream))) return st;
        st = group64_append(L, ki, v + r * krow, 1, pos, stream);
        if (st) return st;
      }
      void* mid = events ? events[3 * r + 1] : nullptr;
      if (events && (st = hip_check(hipEventRecord((hipEvent_t)events[3 * r], s)))) return st;
      st = fused ? decode_fused_append(L, qi, ki, v + r * krow, out + r * qrow, pos, scale,
                                       stream, mid)
                 : group64_attend(L, qi, out + r * qrow, 1, pos, scale, stream, mid);
      if (st) return st;
      if (events && (st = hip_check(hipEventRecord((hipEvent_t)events[3 * r + 2], s)))) return st;
      l++;
    }
  }
  return CIA_OK;
}

extern "C" int cia_decode_loop_ex(cia_layer* layers, int n_layers, const uint16_t* q,
                                  const uint16_t* k, const uint16_t* v, uint16_t* out, int past,
                                  int steps, float scale, int layers_per_launch, void** events,
                                  void* stream) {
  return cia_decode_loop_runs(layers, n_layers, q, k, v, out, past, steps, scale,
                              layers_per_launch, 0, events, stream);
}

extern "C" int cia_decode_loop(cia_layer* layers, int n_layers, const uint16_t* q,
                               const uint16_t* k, const uint16_t* v, uint16_t* out, int past,
                               int steps, float scale, void** events, void* stream) {
  return cia_decode_loop_runs(layers, n_layers, q, k, v, out, past, steps, scale, 0, 0, events,
                              stream);
}

// ---------------------------------------------------------------- attention branch
static int proj_check(const cia_attn_proj* P) {
  if (!P || !P->q_packed || !P->q_scales || !P->k_packed || !P->k_scales || !P->v_packed ||
      !P->v_scales || !P->o_packed || !P->o_scales || !P->ws)
    return CIA_ERR_NULL;
  if (P->cap < 1) return CIA_ERR_ARG;
  return CIA_OK;
}

// engine.cu:792-859 for S tokens; ev (may be NULL) = 4 events as documented
static int attn_block(cia_layer* L, const cia_attn_proj* P, const uint16_t* x, float* h, int S,
                      int past, float scale, int* evicted, void* stream, void* const* ev) {
  constexpr int H = CIA_HIDDEN, NQ = CIA_NH * CIA_HEAD_DIM, NK = CIA_NKV * CIA_HEAD_DIM;
  hipStream_t s = (hipStream_t)stream;
  uint16_t* q = P->ws;
  uint16_t* k = q + (size_t)S * NQ;
  uint16_t* v = k + (size_t)S * NK;
  uint16_t* o = v + (size_t)S * NK;
  int st;
  if (ev && (st = hip_check(hipEventRecord((hipEvent_t)ev[0], s)))) return st;
  if ((st = cia_qkv_proj_int4(x, P->q_packed, P->q_scales, NQ, P->k_packed, P->k_scales,
                              P->v_packed, P->v_scales, NK, H, S, q, k, v, stream)))
    return st;
  if (ev && (st = hip_check(hipEventRecord((hipEvent_t)ev[1], s)))) return st;
  if ((st = cia_layer_forward(L, q, k, v, o, S, past, scale, evicted, stream))) return st;
  if (ev && (st = hip_check(hipEventRecord((hipEvent_t)ev[2], s)))) return st;
  if ((st = cia_gemv_int4_add(o, P->o_packed, P->o_scales, h, H, NQ, S, stream))) return st;
  if (ev && (st = hip_check(hipEventRecord((hipEvent_t)ev[3], s)))) return st;
  return CIA_OK;
}

extern "C" int cia_attn_block_forward(cia_layer* L, const cia_attn_proj* P, const uint16_t* x,
                                      float* h, int S, int past, float scale, int* evicted,
                                      void* stream) {
  if (!L || !x || !h) return CIA_ERR_NULL;
  int st = proj_check(P);
  if (st) return st;
  if (S < 1 || past < 0 || S > P->cap) return CIA_ERR_ARG;
  return attn_block(L, P, x, h, S, past, scale, evicted, stream, nullptr);
}

extern "C" int cia_attn_block_loop(cia_layer* layers, const cia_attn_proj* proj, int n_layers,
                                   const uint16_t* x, float* h, int past, int steps, float scale,
                                   void** events, void* stream) {
  if (!layers || !proj || !x || !h) return CIA_ERR_NULL;
  if (n_layers < 1 || steps < 0 || past < 0) return CIA_ERR_ARG;
  for (int l = 0; l < n_layers; l++) {
    int st = proj_check(&proj[l]);
    if (st) return st;
    if ((st = prep_check(&layers[l]))) return st;
  }
  for (int i = 0; i < steps; i++)
    for (int l = 0; l < n_layers; l++) {
      const size_t r = (size_t)i * n_layers + l;
      const int st = attn_block(&layers[l], &proj[l], x + r * CIA_HIDDEN, h, 1, past + i, scale,
                                nullptr, stream, events ? events + 4 * r : nullptr);
      if (st) return st;
    }
  return CIA_OK;
}
