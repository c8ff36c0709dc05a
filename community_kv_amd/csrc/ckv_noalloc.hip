// ckv_decode_layer_static: ckv_decode_layer with its scratch memory (scores,
// descriptors, slot table, the fused launch's exchange row and counters,
// split partials, per-slot scores, nearest-centroid minima) taken from a
// file-scope device array instead of a caller workspace.  For callers that
// cannot allocate (code under graph capture, serving loops that forbid
// hipMalloc); the caller still passes the state, the KV cache and the outputs.
//
// The array lives once per GPU until the process ends.  Every call on a GPU
// shares it and it keeps the last call's contents: calls that overlap on one
// GPU (two streams, two host threads) race and must not be issued.  The fused
// launch's counters and epoch-tagged exchange row must start at zero for a
// given layout (retrieval heads, community capacity, score coverage and their
// place in the array).  The array's first 256 bytes hold the key of the
// layout that last used it, on the device: every call first launches a
// one-workgroup kernel that compares that key with its own and, when they
// differ, zeroes the exchange row and counters and stores the new key.  The
// decision is therefore taken in stream order on the device, so eager calls,
// captured calls and their replays can be mixed in any order, and a launch
// that fails leaves the stored key unchanged (no memset node: the call stays
// capturable).
#include <mutex>

#include "ckv_device.h"
#include "ckv_error.h"

namespace {

// 16 MiB: e.g. 8 retrieval heads x 8192 communities with a 8192-slot table and
// 32 query heads, or 32 x 2048 with 4096 slots (ckv_decode_static_scratch_bytes).
constexpr size_t SCRATCH_BYTES = (size_t)16 << 20;
constexpr int MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr size_t KEY_BYTES = 256;   // the layout key at the start of the array
constexpr int KEY_WORDS = 6;

std::mutex g_mutex;
unsigned char* g_ptr[MAX_DEVICES] = {};   // device address of `scratch` per GPU

struct LayoutKey {
  uint32_t w[KEY_WORDS];
};

// One workgroup: compare the stored key, clear the exchange row and counters
// (`vecs` 16-byte words) when it differs, then store the new key.  A key word
// is never zero (heads, capacity and coverage are positive), so the zeroed
// array of a fresh process never matches.
__global__ void __launch_bounds__(1024) clear_on_layout_change_kernel(uint32_t* __restrict__ key, LayoutKey now,
                                                                        uint4* __restrict__ region, int64_t vecs) {
  __shared__ int differ;
  if (threadIdx.x == 0) {
    int d = 0;
    for (int i = 0; i < KEY_WORDS; ++i) d |= key[i] != now.w[i];
    differ = d;
  }
  __syncthreads();
  if (differ) {
    for (int64_t i = threadIdx.x; i < vecs; i += blockDim.x) region[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    if (threadIdx.x < KEY_WORDS) key[threadIdx.x] = now.w[threadIdx.x];
  }
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspace capacities the Python layer would allocate for this call
// (attention/kernels/centroid_selection.py: CentroidSelectionWorkspace).
struct Layout {
  int dcap, slot_cap, budget_tiles, score_blocks, tiles;
  size_t off[15];
  size_t total;
};

Layout layout_of(const ckv_graph_state* st, const ckv_decode_config* cfg, int query_heads) {
  Layout l;
  const int R = st->retrieval_heads;
  const int C = st->community_capacity;
  const int inc = cfg->include_current ? 1 : 0;
  l.dcap = cfg->selection_mode == CKV_SELECT_BUDGET ? std::min(cfg->max_selected, C)
                                                    : std::min(cfg->topk_communities, C);
  if (l.dcap < 1) l.dcap = 1;
  const int slots = cfg->num_sink + cfg->max_selected + cfg->local_window + inc;
  l.slot_cap = (slots + CKV_TILE - 1) / CKV_TILE * CKV_TILE;
  l.budget_tiles = cfg->token_budget / CKV_TILE;
  l.score_blocks = (cfg->score_coverage + CKV_SCORE_BLOCK - 1) / CKV_SCORE_BLOCK;
  l.tiles = l.slot_cap / CKV_TILE;
  const size_t sizes[15] = {
      (size_t)R * C * 2,                          // scores
      (size_t)R * l.dcap * 4,                     // communities
      (size_t)R * l.dcap * 4,                     // cumulative ends
      (size_t)R * 4,                              // descriptor counts
      (size_t)R * std::max(l.budget_tiles, 1) * 4,  // tile descriptors
      (size_t)R * 4,                              // selected counts
      (size_t)R * l.slot_cap * 4,                 // slot positions
      (size_t)R * ckv::ckv_exchange_words(C) * 8,  // exchange
      (size_t)R * 4,                              // nearest
      (size_t)R * 4 * 4,                          // block counters
      (size_t)query_heads * l.tiles * 4,          // partial max
      (size_t)query_heads * l.tiles * 4,          // partial sum
      (size_t)query_heads * l.tiles * CKV_HEAD_DIM * 4,  // partial accumulators
      (size_t)R * l.slot_cap * 4,                 // slot scores
      0};
  size_t at = KEY_BYTES;
  for (int i = 0; i < 15; ++i) {
    l.off[i] = at;
    at += align256(sizes[i]);
  }
  l.total = at;
  return l;
}

}  // namespace

extern "C" size_t ckv_decode_static_scratch_bytes(const ckv_graph_state* st, const ckv_decode_config* cfg,
                                                  int32_t query_heads) {
  if (!st || !cfg || query_heads <= 0 || st->retrieval_heads <= 0 || st->community_capacity <= 0) return 0;
  return layout_of(st, cfg, query_heads).total;
}

extern "C" size_t ckv_decode_static_scratch_limit(void) { return SCRATCH_BYTES; }

extern "C" int ckv_decode_layer_static(const ckv_kv_cache* kv, const ckv_graph_state* st,
                                       const ckv_prefill_csr* csr, const ckv_delta_chunks* dl,
                                       const ckv_decode_config* cfg, void* output, float* lse, float* topk_scores,
                                       int32_t* topk_positions, int32_t* assigned, int32_t* overflow,
                                       void* stream) {
  if (!kv || !st || !csr || !dl || !cfg) return ckv_internal::set_error(CKV_E_INVALID, "null argument struct");
  if (st->retrieval_heads <= 0 || st->community_capacity <= 0 || kv->query_heads <= 0)
    return ckv_internal::set_error(CKV_E_INVALID, "empty graph state");
  if (cfg->token_budget <= 0 || cfg->token_budget % CKV_TILE || cfg->max_selected < 0 || cfg->num_sink < 0 ||
      cfg->local_window < 0 || cfg->score_coverage <= 0)
    return ckv_internal::set_error(CKV_E_INVALID, "token budget, slot counts or score coverage out of range");
  const Layout l = layout_of(st, cfg, kv->query_heads);
  if (l.total > SCRATCH_BYTES)
    return ckv_internal::set_error(CKV_E_LIMIT,
                                   "the layer needs more scratch than the static decode scratch holds (16 MiB; "
                                   "ckv_decode_static_scratch_bytes gives the need): use ckv_decode_layer");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return ckv_internal::set_error(CKV_E_LAUNCH, "no current HIP device");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  unsigned char* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_ptr[dev] == nullptr) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        return ckv_internal::set_error(CKV_E_LAUNCH, "hipGetSymbolAddress of the static decode scratch failed");
      }
      g_ptr[dev] = static_cast<unsigned char*>(p);
    }
    base = g_ptr[dev];
  }
  ckv_decode_workspace ws;
  ws.scores = reinterpret_cast<uint16_t*>(base + l.off[0]);
  ws.communities = reinterpret_cast<int32_t*>(base + l.off[1]);
  ws.cumulative_ends = reinterpret_cast<int32_t*>(base + l.off[2]);
  ws.descriptor_counts = reinterpret_cast<int32_t*>(base + l.off[3]);
  ws.tile_descriptors = reinterpret_cast<int32_t*>(base + l.off[4]);
  ws.selected_counts = reinterpret_cast<int32_t*>(base + l.off[5]);
  ws.slot_positions = reinterpret_cast<int32_t*>(base + l.off[6]);
  ws.exchange = reinterpret_cast<uint64_t*>(base + l.off[7]);
  ws.nearest = reinterpret_cast<int32_t*>(base + l.off[8]);
  ws.block_counters = reinterpret_cast<uint32_t*>(base + l.off[9]);
  ws.partial_max = reinterpret_cast<float*>(base + l.off[10]);
  ws.partial_sum = reinterpret_cast<float*>(base + l.off[11]);
  ws.partial_acc = reinterpret_cast<float*>(base + l.off[12]);
  ws.slot_scores = reinterpret_cast<float*>(base + l.off[13]);
  ws.output = output;
  ws.lse = lse;
  ws.topk_scores = topk_scores;
  ws.topk_positions = topk_positions;
  ws.assigned = assigned;
  ws.overflow = overflow;
  ws.descriptor_capacity = l.dcap;
  ws.slot_capacity = l.slot_cap;
  ws.budget_tiles = l.budget_tiles;
  ws.score_blocks = l.score_blocks;
  {
    // exchange row and block counters are contiguous (256-byte aligned): zero both on a layout change.
    // The score coverage is part of the key because the fused and the multi-kernel selections write the
    // nearest-centroid words of the exchange row in different formats.
    const LayoutKey now{{(uint32_t)st->retrieval_heads, (uint32_t)st->community_capacity,
                         (uint32_t)cfg->score_coverage, (uint32_t)l.off[7], (uint32_t)l.off[10],
                         (uint32_t)kv->query_heads}};
    const int64_t vecs = (int64_t)(l.off[10] - l.off[7]) / 16;
    hipLaunchKernelGGL(clear_on_layout_change_kernel, dim3(1), dim3(1024), 0, s, reinterpret_cast<uint32_t*>(base),
                       now, reinterpret_cast<uint4*>(base + l.off[7]), vecs);
    const int rc = ckv::launch_check("static scratch clear");
    if (rc) return rc;
  }
  return ckv_decode_layer(kv, st, csr, dl, cfg, &ws, stream);
}
