// C ABI of libckv_amd.so (include/ckv_amd.h): argument validation, error
// reporting and the decode entry points.  Kernels live in ckv_select.hip
// (scoring + selection + slot table), ckv_attend.hip (attention, split merge,
// online update, dense baseline) and ckv_prefill.hip (prefill edge export).
//
// ckv_decode_layer is three stream-ordered launches when the layer fits the
// fused path (bf16 KV with prefill membership, slot table <= 8192, group
// <= 4): select_attend_kernel (selection + attention partials), the split
// merge, and the online update (callers that defer it fold it into the next
// layer's launch: ckv_decode_step_after_update).  Otherwise: select_kernel,
// the attention partials kernel, the merge and the update.  A layer-wise shared
// graph adds the centroid sync after the update.  ckv_state.hip builds the
// prefill state from labels.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "ckv_device.h"
#include "ckv_error.h"

namespace {

constexpr int64_t FUSED_MAX_WORKGROUPS = 256;  // compute units of the MI355X

thread_local char g_error[512] = "";

int fail(int code, const char* message) {
  snprintf(g_error, sizeof(g_error), "%s", message);
  return code;
}

int validate(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
             const ckv_delta_chunks* dl, const ckv_decode_config* cfg, const ckv_decode_workspace* ws) {
  if (!kv || !st || !csr || !dl || !cfg || !ws) return fail(CKV_E_INVALID, "null argument struct");
  if (!kv->query || !kv->key || !kv->value) return fail(CKV_E_INVALID, "null query/key/value");
  if (kv->dtype != CKV_BF16 && kv->dtype != CKV_F32) return fail(CKV_E_INVALID, "kv dtype must be bf16 or f32");
  if (st->centroid_dtype != CKV_E4M3 && st->centroid_dtype != CKV_F32)
    return fail(CKV_E_INVALID, "centroid dtype must be e4m3 or f32");
  if (cfg->group_size < 1 || cfg->group_size > CKV_MAX_GROUP)
    return fail(CKV_E_INVALID, "group_size must be in [1, 16]");
  if (st->retrieval_heads <= 0 || st->graph_count <= 0 || st->community_capacity <= 0)
    return fail(CKV_E_INVALID, "empty graph state");
  if (!st->centroids || !st->community_sizes || !st->community_counts || !st->retrieval_to_graph ||
      !st->retrieval_to_kv || !st->current_position)
    return fail(CKV_E_INVALID, "incomplete graph state");
  if (st->retrieval_heads * cfg->group_size != kv->query_heads)
    return fail(CKV_E_INVALID, "query heads must equal retrieval heads x group size");
  if (st->community_capacity > CKV_MAX_COMMUNITIES) return fail(CKV_E_LIMIT, "community capacity exceeds 65536");
  if (ws->descriptor_capacity <= 0 || ws->descriptor_capacity > CKV_MAX_DESCRIPTORS)
    return fail(CKV_E_LIMIT, "descriptor capacity must be in [1, 4096]");
  if (ws->slot_capacity <= 0 || ws->slot_capacity % CKV_TILE || ws->slot_capacity > 2048 * CKV_TILE)
    return fail(CKV_E_INVALID, "slot capacity must be a positive multiple of 64, at most 131072");
  if (cfg->num_sink < 0 || cfg->max_selected < 0 || cfg->local_window < 0)
    return fail(CKV_E_INVALID, "negative slot counts");
  if (cfg->num_sink > CKV_MAX_SINKS) return fail(CKV_E_LIMIT, "num_sink exceeds 256");
  if (cfg->local_window > CKV_MAX_WINDOW) return fail(CKV_E_LIMIT, "local_window exceeds 1024");
  if (cfg->num_sink + cfg->max_selected + cfg->local_window + (cfg->include_current ? 1 : 0) > ws->slot_capacity)
    return fail(CKV_E_INVALID, "slot capacity smaller than sinks + selected + window + current");
  if (csr->member_offsets && cfg->num_sink > 0 && !cfg->sink_positions)
    return fail(CKV_E_INVALID, "null sink positions");
  if (csr->member_offsets && (!csr->member_positions || !dl->positions || !dl->chunk_start || !dl->chunk_size ||
                              !dl->chunk_previous || !dl->community_tail || !dl->community_sizes ||
                              !st->token_communities))
    return fail(CKV_E_INVALID, "incomplete membership / delta-chunk state");
  if (cfg->selection_mode != CKV_SELECT_BUDGET && cfg->selection_mode != CKV_SELECT_TOPK)
    return fail(CKV_E_INVALID, "unknown selection mode");
  if (cfg->selection_mode == CKV_SELECT_TOPK && cfg->topk_communities <= 0)
    return fail(CKV_E_INVALID, "topk_communities must be positive");
  if (cfg->assignment < CKV_ASSIGN_NONE || cfg->assignment > CKV_ASSIGN_NEAREST)
    return fail(CKV_E_INVALID, "unknown assignment mode");
  if (cfg->score_coverage <= 0 || cfg->score_coverage > st->community_capacity)
    return fail(CKV_E_INVALID, "score coverage must be in [1, community capacity]");
  if (ws->score_blocks != (cfg->score_coverage + CKV_SCORE_BLOCK - 1) / CKV_SCORE_BLOCK)
    return fail(CKV_E_INVALID, "score_blocks must equal ceil(score_coverage / 64)");
  if (!ws->scores || !ws->communities || !ws->cumulative_ends || !ws->descriptor_counts || !ws->tile_descriptors ||
      !ws->selected_counts || !ws->slot_positions || !ws->block_counters ||
      (cfg->assignment == CKV_ASSIGN_NEAREST && !ws->nearest))
    return fail(CKV_E_INVALID, "selection workspace is incomplete");
  if (kv->head_stride % 8 || kv->token_stride % 8)
    return fail(CKV_E_INVALID, "kv strides must be multiples of 8 elements");
  return CKV_OK;
}

int validate_attention(const ckv_graph_state* st, const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                       const ckv_decode_workspace* ws) {
  if (!ws->partial_max || !ws->partial_sum || !ws->partial_acc || !ws->output || !ws->lse)
    return fail(CKV_E_INVALID, "attention workspace is incomplete");
  if (cfg->assignment != CKV_ASSIGN_NONE &&
      (!ws->slot_scores || !ws->topk_scores || !ws->topk_positions || !ws->assigned || !ws->overflow ||
       !st->token_communities || !st->community_weight || !st->total_weight || !dl->positions ||
       !dl->chunk_start || !dl->chunk_capacity || !dl->chunk_size || !dl->chunk_next || !dl->chunk_previous ||
       !dl->community_head || !dl->community_tail || !dl->community_sizes || !dl->next_free_chunk ||
       !dl->next_free_position))
    return fail(CKV_E_INVALID, "update state or workspace is incomplete");
  return CKV_OK;
}

ckv::DecodeArgs pack(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                     const ckv_delta_chunks* dl, const ckv_decode_config* cfg, const ckv_decode_workspace* ws) {
  ckv::DecodeArgs a;
  a.kv = *kv;
  a.st = *st;
  a.csr = *csr;
  a.dl = *dl;
  a.cfg = *cfg;
  a.ws = *ws;
  return a;
}

}  // namespace

int ckv_internal::set_error(int code, const char* message) { return fail(code, message); }

int ckv::launch_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_error, sizeof(g_error), "%s launch failed: %s", what, hipGetErrorString(e));
    return CKV_E_LAUNCH;
  }
  return CKV_OK;
}

extern "C" int ckv_abi_version(void) { return CKV_ABI_VERSION; }

extern "C" const char* ckv_last_error(void) { return g_error; }

extern "C" int ckv_host_numerics(int op, const float* in, void* out, int64_t n) {
  if (!in || !out || n < 0) return fail(CKV_E_INVALID, "null argument");
  for (int64_t i = 0; i < n; ++i) {
    switch (op) {
      case 0: reinterpret_cast<float*>(out)[i] = ckv_expf(in[i]); break;
      case 1: reinterpret_cast<float*>(out)[i] = ckv_logf(in[i]); break;
      case 2: reinterpret_cast<uint16_t*>(out)[i] = ckv_f32_to_f16_bits(in[i]); break;
      case 3: reinterpret_cast<uint16_t*>(out)[i] = ckv_f32_to_bf16_bits(in[i]); break;
      case 4: reinterpret_cast<uint8_t*>(out)[i] = ckv_f32_to_e4m3(in[i]); break;
      case 5: reinterpret_cast<float*>(out)[i] = ckv_e4m3_to_f32((uint8_t)in[i]); break;
      default: return fail(CKV_E_INVALID, "unknown numerics op");
    }
  }
  return CKV_OK;
}

extern "C" int ckv_score_select(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                                const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                                ckv_decode_workspace* ws, void* stream) {
  const int rc = validate(kv, st, csr, dl, cfg, ws);
  if (rc) return rc;
  return ckv::launch_score_select(pack(kv, st, csr, dl, cfg, ws), reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckv_segmented_attention(const ckv_kv_cache* kv, const ckv_graph_state* st,
                                       const ckv_prefill_csr* csr, const ckv_delta_chunks* dl,
                                       const ckv_decode_config* cfg, ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (!rc) rc = validate_attention(st, dl, cfg, ws);
  if (rc) return rc;
  return ckv::launch_attention(pack(kv, st, csr, dl, cfg, ws), reinterpret_cast<hipStream_t>(stream), false);
}

extern "C" int ckv_attention_partials(const ckv_kv_cache* kv, const ckv_graph_state* st,
                                      const ckv_prefill_csr* csr, const ckv_delta_chunks* dl,
                                      const ckv_decode_config* cfg, ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (!rc) rc = validate_attention(st, dl, cfg, ws);
  if (rc) return rc;
  return ckv::launch_attention(pack(kv, st, csr, dl, cfg, ws), reinterpret_cast<hipStream_t>(stream), true);
}

// Parts per head of the fused launch for one layer, or 0 for the separate
// selection, attention and merge launches: the cooperative launch shares the
// scoring between a head's parts; without it every fused workgroup repeats
// its head's whole selection, worth it only while the copies run side by
// side, one per compute unit (with 32 per-query-head graphs and a 4,096-token
// budget, 1,024 workgroups would run four rounds of full selections).
static int single_fused_parts(const ckv::DecodeArgs& a) {
  const int parts = ckv::fused_parts(a);
  if (parts > 0 && ckv::coop_parts(a) == 0 && (int64_t)a.st.retrieval_heads * parts > FUSED_MAX_WORKGROUPS) return 0;
  return parts;
}

extern "C" int ckv_decode_layer(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                                const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                                ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (!rc) rc = validate_attention(st, dl, cfg, ws);
  if (rc) return rc;
  const ckv::DecodeArgs a = pack(kv, st, csr, dl, cfg, ws);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int parts = single_fused_parts(a);
  if (ckv::coop_parts(a) > 0) {  // merged inside the launch; the update follows
    rc = ckv::launch_select_attend(a, s, nullptr, parts, true);
    return rc ? rc : ckv::launch_update(a, s);
  }
  if (parts > 0) {
    rc = ckv::launch_select_attend(a, s, nullptr, parts, false);
    return rc ? rc : ckv::launch_merge_update(a, s, parts);
  }
  rc = ckv::launch_score_select(a, s);
  if (!rc) rc = ckv::launch_attention(a, s, false);
  if (!rc) rc = ckv::launch_update(a, s);
  return rc;
}

extern "C" int ckv_score_select_after_update(const ckv_layer_args* layer, const ckv_layer_args* pending,
                                             void* stream) {
  if (!layer) return fail(CKV_E_INVALID, "null layer arguments");
  int rc = validate(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  if (rc) return rc;
  const ckv::DecodeArgs a = pack(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!pending) return ckv::launch_score_select(a, s);
  rc = validate(pending->kv, pending->state, pending->csr, pending->deltas, pending->config, pending->ws);
  if (!rc) rc = validate_attention(pending->state, pending->deltas, pending->config, pending->ws);
  if (rc) return rc;
  if (pending->state->centroids == layer->state->centroids || pending->ws->lse == layer->ws->lse)
    return fail(CKV_E_INVALID, "the pending update must belong to another layer");
  const ckv::DecodeArgs u =
      pack(pending->kv, pending->state, pending->csr, pending->deltas, pending->config, pending->ws);
  if (u.st.centroid_dtype != a.st.centroid_dtype || u.kv.dtype != a.kv.dtype) {
    rc = ckv::launch_update(u, s);  // different dtypes: a launch of its own, before the selection
    return rc ? rc : ckv::launch_score_select(a, s);
  }
  rc = ckv::launch_score_select(a, s, &u);
  return rc ? rc : ckv::launch_sync_shared(u, s);
}

extern "C" int ckv_decode_step_after_update(const ckv_layer_args* layer, const ckv_layer_args* pending,
                                            void* stream) {
  if (!layer) return fail(CKV_E_INVALID, "null layer arguments");
  int rc = validate(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  if (!rc) rc = validate_attention(layer->state, layer->deltas, layer->config, layer->ws);
  if (rc) return rc;
  const ckv::DecodeArgs a = pack(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int parts = single_fused_parts(a);
  if (parts == 0) {
    rc = ckv_score_select_after_update(layer, pending, stream);
    return rc ? rc : ckv::launch_attention(a, s, false);
  }
  ckv::DecodeArgs u;
  const ckv::DecodeArgs* up = nullptr;
  if (pending) {
    rc = validate(pending->kv, pending->state, pending->csr, pending->deltas, pending->config, pending->ws);
    if (!rc) rc = validate_attention(pending->state, pending->deltas, pending->config, pending->ws);
    if (rc) return rc;
    if (pending->state->centroids == layer->state->centroids || pending->ws->lse == layer->ws->lse)
      return fail(CKV_E_INVALID, "the pending update must belong to another layer");
    u = pack(pending->kv, pending->state, pending->csr, pending->deltas, pending->config, pending->ws);
    if (u.st.centroid_dtype != a.st.centroid_dtype || u.kv.dtype != a.kv.dtype) {
      rc = ckv::launch_update(u, s);  // different dtypes: a launch of its own, before this layer
      if (rc) return rc;
    } else {
      up = &u;
    }
  }
  const bool coop = ckv::coop_parts(a) > 0;
  rc = ckv::launch_select_attend(a, s, up, parts, coop);
  if (!rc && up) rc = ckv::launch_sync_shared(u, s);
  if (!rc && !coop) rc = ckv::launch_merge(a, s, parts);
  return rc;
}

extern "C" int ckv_online_update(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                                 const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                                 ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (!rc) rc = validate_attention(st, dl, cfg, ws);
  if (rc) return rc;
  return ckv::launch_update(pack(kv, st, csr, dl, cfg, ws), reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckv_dense_decode(const ckv_kv_cache* kv, int32_t seq_len, float softmax_scale, float* partial_max,
                                float* partial_sum, float* partial_acc, void* output, float* lse, void* stream) {
  if (!kv || !kv->query || !kv->key || !kv->value || !partial_max || !partial_sum || !partial_acc || !output || !lse)
    return fail(CKV_E_INVALID, "null argument");
  if (kv->kv_heads <= 0 || kv->query_heads % kv->kv_heads)
    return fail(CKV_E_INVALID, "query heads must be a multiple of kv heads");
  const int group = kv->query_heads / kv->kv_heads;
  if (group > CKV_MAX_GROUP) return fail(CKV_E_INVALID, "group size exceeds 16");
  if (seq_len <= 0 || seq_len > kv->capacity || seq_len > 2048 * CKV_TILE)
    return fail(CKV_E_INVALID, "seq_len out of range (at most 131072)");
  if (kv->dtype != CKV_BF16 && kv->dtype != CKV_F32) return fail(CKV_E_INVALID, "kv dtype must be bf16 or f32");
  if (kv->head_stride % 8 || kv->token_stride % 8)
    return fail(CKV_E_INVALID, "kv strides must be multiples of 8 elements");
  ckv::DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.kv = *kv;
  a.cfg.softmax_scale = softmax_scale;
  a.cfg.group_size = group;
  a.ws.partial_max = partial_max;
  a.ws.partial_sum = partial_sum;
  a.ws.partial_acc = partial_acc;
  a.ws.output = output;
  a.ws.lse = lse;
  return ckv::launch_dense(a, seq_len, group, reinterpret_cast<hipStream_t>(stream));
}

namespace {

// Checks a batch and returns the launch maxima.  Every item must pass the
// single-call checks, use bf16 KV, and share the first item's centroid dtype,
// group size, retrieval heads, slot capacity and assignment mode; items must
// not share state or workspace.
int validate_batch(const ckv_layer_args* items, int count, std::vector<ckv::DecodeArgs>* packed, int* max_nscore,
                   size_t* max_lds, bool* any_shared, size_t* max_large_lds) {
  if (!items || count <= 0) return fail(CKV_E_INVALID, "empty batch");
  *max_nscore = 0;
  *max_lds = 0;
  *max_large_lds = 0;
  *any_shared = false;
  for (int i = 0; i < count; ++i) {
    const ckv_layer_args& it = items[i];
    int rc = validate(it.kv, it.state, it.csr, it.deltas, it.config, it.ws);
    if (!rc) rc = validate_attention(it.state, it.deltas, it.config, it.ws);
    if (rc) return rc;
    const ckv::DecodeArgs a = pack(it.kv, it.state, it.csr, it.deltas, it.config, it.ws);
    if (a.kv.dtype != CKV_BF16) return fail(CKV_E_INVALID, "batched decode requires bf16 KV");
    if (std::min(a.st.community_capacity, a.ws.score_blocks * CKV_SCORE_BLOCK) > CKV_MAX_COMMUNITIES)
      return fail(CKV_E_LIMIT, "batched decode scores at most 65536 communities per head");
    if (a.cfg.assignment == CKV_ASSIGN_NEAREST && a.ws.exchange == nullptr &&
        std::min(a.st.community_capacity, a.ws.score_blocks * CKV_SCORE_BLOCK) > CKV_MAX_SELECT_ROWS)
      return fail(CKV_E_LIMIT, "nearest-centroid assignment above 8192 scored communities needs the exchange workspace");
    if (ckv::attention_batch_splits(a) == 0)
      return fail(CKV_E_LIMIT, "batched decode requires group_size * 128 <= 512 and at most 64 attention splits");
    if (i > 0) {
      const ckv::DecodeArgs& h = (*packed)[0];
      if (a.st.centroid_dtype != h.st.centroid_dtype || a.cfg.group_size != h.cfg.group_size ||
          a.st.retrieval_heads != h.st.retrieval_heads || a.ws.slot_capacity != h.ws.slot_capacity ||
          a.cfg.assignment != h.cfg.assignment)
        return fail(CKV_E_INVALID, "batch items must share dtypes, group size, heads, slot capacity and assignment");
      for (const ckv::DecodeArgs& o : *packed) {
        if (o.st.centroids == a.st.centroids || o.ws.lse == a.ws.lse || o.ws.slot_positions == a.ws.slot_positions)
          return fail(CKV_E_INVALID, "batch items must not share state or workspace");
      }
    }
    packed->push_back(a);
    *max_nscore = std::max(*max_nscore, std::min(a.st.community_capacity, a.ws.score_blocks * CKV_SCORE_BLOCK));
    *max_lds = std::max(*max_lds, ckv::select_lds_bytes(std::min(a.st.community_capacity,
                                                                 a.ws.score_blocks * CKV_SCORE_BLOCK),
                                                        a.ws.descriptor_capacity, a.cfg.max_selected));
    *max_large_lds = std::max(*max_large_lds, ckv::select_large_lds_bytes(a));
    if (a.st.retrieval_heads != a.st.graph_count) *any_shared = true;
  }
  return CKV_OK;
}

}  // namespace

extern "C" size_t ckv_batch_table_bytes(int32_t count) {
  return count > 0 ? (size_t)count * sizeof(ckv::DecodeArgs) : 0;
}

extern "C" int ckv_batch_prepare(const ckv_layer_args* items, int32_t count, void* table, void* stream) {
  std::vector<ckv::DecodeArgs> packed;
  int max_nscore;
  size_t max_lds;
  bool any_shared;
  size_t max_large_lds;
  const int rc = validate_batch(items, count, &packed, &max_nscore, &max_lds, &any_shared, &max_large_lds);
  if (rc) return rc;
  if (!table) return fail(CKV_E_INVALID, "null batch table");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(table, packed.data(), packed.size() * sizeof(ckv::DecodeArgs), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail(CKV_E_LAUNCH, hipGetErrorString(e));
  return CKV_OK;
}

namespace {

// One batched step of `items`; `defer`: leave the items' online update
// pending (the split merge alone ends the step).  `pending` (null: none): a
// batch whose update is pending, run in extra workgroups of the selection
// launch where the selection path has them, else in a launch of its own
// before the step.
int batch_step(const ckv_layer_args* items, int32_t count, const void* table, const ckv_layer_args* pending,
               int32_t pending_count, const void* pending_table, bool defer, void* stream) {
  std::vector<ckv::DecodeArgs> packed;
  int max_nscore;
  size_t max_lds;
  bool any_shared;
  size_t max_large_lds;
  int rc = validate_batch(items, count, &packed, &max_nscore, &max_lds, &any_shared, &max_large_lds);
  if (rc) return rc;
  if (!table) return fail(CKV_E_INVALID, "null batch table");
  const ckv::DecodeArgs* t = reinterpret_cast<const ckv::DecodeArgs*>(table);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const ckv::DecodeArgs& h = packed[0];

  std::vector<ckv::DecodeArgs> upacked;
  bool u_shared = false;
  const ckv::DecodeArgs* ut = nullptr;
  if (pending) {
    int u_nscore;
    size_t u_lds, u_large;
    rc = validate_batch(pending, pending_count, &upacked, &u_nscore, &u_lds, &u_shared, &u_large);
    if (rc) return rc;
    if (!pending_table) return fail(CKV_E_INVALID, "null pending batch table");
    for (const ckv::DecodeArgs& u : upacked) {
      for (const ckv::DecodeArgs& it : packed) {
        if (u.st.centroids == it.st.centroids || u.ws.lse == it.ws.lse || u.ws.slot_positions == it.ws.slot_positions)
          return fail(CKV_E_INVALID, "the pending batch must not share state or workspace with this batch");
      }
    }
    if (upacked[0].cfg.assignment != CKV_ASSIGN_NONE) ut = reinterpret_cast<const ckv::DecodeArgs*>(pending_table);
  }

  int parts = ckv::fused_parts(h);
  size_t fused_lds = 0;
  for (const ckv::DecodeArgs& it : packed) {
    if (ckv::fused_parts(it) != parts) parts = 0;
    fused_lds = std::max(fused_lds, ckv::fused_lds_bytes(it));
  }
  // Every fused workgroup repeats its head's selection: worth it only while
  // the copies run side by side, one per compute unit.
  if ((int64_t)count * h.st.retrieval_heads * parts > FUSED_MAX_WORKGROUPS) parts = 0;
  // above 8,192 scored rows (one workgroup's registers) the whole batch takes
  // the large selection: scoring on every compute unit, 1,024 threads per head
  const bool large = max_nscore > CKV_MAX_SELECT_ROWS;
  if (large) parts = 0;
  const bool ride = ut != nullptr && parts == 0 && !large && upacked[0].st.centroid_dtype == h.st.centroid_dtype;
  if (ut != nullptr && !ride) {  // the pending update in a launch of its own
    rc = ckv::launch_batch_update(upacked[0], ut, pending_count, u_shared, s);
    if (rc) return rc;
  }
  int splits = parts;
  if (parts > 0) {
    rc = ckv::launch_batch_select_attend(h, t, count, max_nscore, fused_lds, parts, s);
  } else {
    if (large) {
      rc = ckv::launch_batch_select_large(h, t, count, max_nscore, max_large_lds, s);
    } else if (ride) {
      rc = ckv::launch_batch_select(h, t, count, max_nscore, max_lds, s, ut, pending_count,
                                    upacked[0].st.retrieval_heads);
      if (!rc && u_shared) rc = ckv::launch_batch_sync_shared(upacked[0], ut, pending_count, s);
    } else {
      rc = ckv::launch_batch_select(h, t, count, max_nscore, max_lds, s);
    }
    if (!rc) rc = ckv::launch_batch_attention(h, t, count, s, true);
    splits = ckv::attention_batch_splits(h);
  }
  if (rc) return rc;
  if (defer || h.cfg.assignment == CKV_ASSIGN_NONE) return ckv::launch_batch_merge(h, t, count, splits, s);
  return ckv::launch_batch_merge_update(h, t, count, splits, any_shared, s);
}

}  // namespace

extern "C" int ckv_batch_decode(const ckv_layer_args* items, int32_t count, const void* table, void* stream) {
  return batch_step(items, count, table, nullptr, 0, nullptr, false, stream);
}

extern "C" int ckv_batch_decode_after_update(const ckv_layer_args* items, int32_t count, const void* table,
                                             const ckv_layer_args* pending, int32_t pending_count,
                                             const void* pending_table, void* stream) {
  return batch_step(items, count, table, pending, pending_count, pending_table, true, stream);
}

extern "C" int ckv_batch_online_update(const ckv_layer_args* items, int32_t count, const void* table, void* stream) {
  std::vector<ckv::DecodeArgs> packed;
  int max_nscore;
  size_t max_lds;
  bool any_shared;
  size_t max_large_lds;
  const int rc = validate_batch(items, count, &packed, &max_nscore, &max_lds, &any_shared, &max_large_lds);
  if (rc) return rc;
  if (!table) return fail(CKV_E_INVALID, "null batch table");
  if (packed[0].cfg.assignment == CKV_ASSIGN_NONE) return CKV_OK;
  return ckv::launch_batch_update(packed[0], reinterpret_cast<const ckv::DecodeArgs*>(table), count, any_shared,
                                  reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckv_batch_attention_partials(const ckv_layer_args* items, int32_t count, const void* table,
                                            void* stream) {
  std::vector<ckv::DecodeArgs> packed;
  int max_nscore;
  size_t max_lds;
  bool any_shared;
  size_t max_large_lds;
  const int rc = validate_batch(items, count, &packed, &max_nscore, &max_lds, &any_shared, &max_large_lds);
  if (rc) return rc;
  if (!table) return fail(CKV_E_INVALID, "null batch table");
  return ckv::launch_batch_attention(packed[0], reinterpret_cast<const ckv::DecodeArgs*>(table), count,
                                     reinterpret_cast<hipStream_t>(stream), true);
}

extern "C" int ckv_select_attend_partials(const ckv_layer_args* layer, void* stream) {
  if (!layer) return fail(CKV_E_INVALID, "null layer arguments");
  int rc = validate(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  if (!rc) rc = validate_attention(layer->state, layer->deltas, layer->config, layer->ws);
  if (rc) return rc;
  const ckv::DecodeArgs a = pack(layer->kv, layer->state, layer->csr, layer->deltas, layer->config, layer->ws);
  const int parts = ckv::fused_parts(a);
  if (parts == 0) return fail(CKV_E_INVALID, "the fused selection + attention path cannot serve this layer");
  return ckv::launch_select_attend(a, reinterpret_cast<hipStream_t>(stream), nullptr, parts, false);
}
