/*
 * ckv_amd.h -- C ABI of the MI355X (gfx950) CommunityKV sparse-decode library
 * (libckv_amd.so, built from community_kv_amd/csrc/).
 *
 * Every entry point takes plain device pointers and sizes, never allocates,
 * never synchronises the host, runs on the HIP stream it is given, and returns
 * 0 on success or a nonzero CKV_E* code with a message readable through
 * ckv_last_error().  Tensors are dense row-major; the only strides are those
 * of the KV cache.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   ckv_score_select        score_and_select()                attention/kernels/centroid_selection.py:537-556
 *                           = score_centroids()               attention/kernels/centroid_selection.py:330-445
 *                           + select_weighted_descriptors()   attention/kernels/_csrc/bindings.cpp:3-21,
 *                                                             attention/kernels/_csrc/descriptor_selection.cu:852-1189
 *   ckv_segmented_attention triton_segmented_attention()      attention/kernels/segmented_attention.py:1016-1273
 *                           (partials kernel 31-365, split reduce of the fused reduce+update
 *                            kernel 368-864)
 *   ckv_online_update       the update half of that fused kernel (segmented_attention.py:368-864,
 *                           launched at 1164-1273) and the shared-graph centroid sync 867-950;
 *                           a separate entry point so that callers can run it on another stream
 *   ckv_decode_layer        decode_layer()                    attention/decode.py:67-111
 *   ckv_batch_decode        a loop of decode_layer() over independent sequences (batched launches;
 *                           ckv_batch_prepare is its set-up call and synchronises its stream)
 *   ckv_dense_decode        (baseline only) dense bf16 decode over the whole cache, the
 *                           FlashAttention decode the reference compares against (paper Table 5)
 *   ckv_prefill_attention_topk
 *                           prefill_attention_topk()          attention/flash_attention.py:23-51
 *                           (patched FA3 op, third_party/flash_attention/community-kv.patch:31-120)
 *   ckv_label_counts,       the state build of build_partitioned_layer() after Leiden
 *   ckv_build_layer_state   (graph/partition.py:538-618): compute_centroids 382-454,
 *                           build_member_csr 457-492, init_modularity_state 495-535
 *   ckv_build_adjacency     build_adjacency()                 graph/partition.py:168-249
 *   ckv_batched_leiden      batched_leiden() of the Leiden extension (graph/leiden/_csrc/bindings.cpp:40-103,
 *                           launch_batched_leiden in leiden.cu:43-205), called by run_leiden()
 *                           (graph/leiden/algorithm.py:51-161)
 *   ckv_aggregate_coo       aggregate_coo() of the same extension (bindings.cpp:118-170,
 *                           aggregate_upper_coo in aggregate.cu:88-184)
 *   ckv_densify_count,      _densify_per_graph() (graph/leiden/algorithm.py:30-48), as two calls
 *   ckv_densify_apply       so that the caller reads the per-graph counts in between
 */
#ifndef CKV_AMD_H
#define CKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKV_ABI_VERSION 3
#define CKV_HEAD_DIM 128
#define CKV_TILE 64
#define CKV_KAPPA 8
#define CKV_SCORE_BLOCK 64
#define CKV_MAX_GROUP 16
#define CKV_MAX_COMMUNITIES 65536   /* community capacity per graph state */
#define CKV_MAX_SELECT_ROWS 8192    /* scored rows per head that one selection workgroup holds in registers;
                                       more go through the multi-kernel selection */
#define CKV_MAX_DESCRIPTORS 4096
#define CKV_MAX_SINKS 256
#define CKV_MAX_WINDOW 1024

enum ckv_status {
  CKV_OK = 0,
  CKV_E_INVALID = 1,   /* bad argument: shapes, modes, null pointers */
  CKV_E_LIMIT = 2,     /* a size exceeds a compiled-in limit */
  CKV_E_LAUNCH = 3     /* the HIP runtime reported a launch error */
};

enum ckv_dtype { CKV_BF16 = 0, CKV_F32 = 1, CKV_E4M3 = 2 };
enum ckv_selection_mode { CKV_SELECT_BUDGET = 0, CKV_SELECT_TOPK = 1 };
enum ckv_assignment { CKV_ASSIGN_NONE = 0, CKV_ASSIGN_DELTA_Q = 1, CKV_ASSIGN_NEAREST = 2 };

/* Query and KV cache of one layer (reference: decode_layer query/key/value). */
typedef struct ckv_kv_cache {
  const void* query;        /* [query_heads][128], dtype */
  const void* key;          /* key[h*head_stride + t*token_stride + d] */
  const void* value;        /* same layout as key */
  int64_t head_stride;      /* elements */
  int64_t token_stride;     /* elements */
  int64_t capacity;         /* tokens addressable per head (key.shape[1]) */
  int32_t query_heads;
  int32_t kv_heads;
  int32_t dtype;            /* CKV_BF16 or CKV_F32 */
  int32_t reserved;
} ckv_kv_cache;

/* Immutable prefill membership (reference: PrefillCSR, graph/state.py:15-61). */
typedef struct ckv_prefill_csr {
  const int32_t* member_offsets;    /* [graphs][community_capacity + 1] */
  const int32_t* member_positions;  /* [graphs][member_stride], recency descending */
  int64_t member_stride;
} ckv_prefill_csr;

/* Geometric decode-delta chunks (reference: DecodeDeltaChunks, graph/state.py:64-248). */
typedef struct ckv_delta_chunks {
  int32_t* positions;          /* [graphs][position_capacity] */
  int32_t* chunk_start;        /* [graphs][chunks_per_graph] */
  int32_t* chunk_capacity;
  int32_t* chunk_size;
  int32_t* chunk_next;
  int32_t* chunk_previous;
  int32_t* community_head;     /* [graphs][community_capacity] */
  int32_t* community_tail;
  int32_t* community_sizes;
  int32_t* next_free_chunk;    /* [graphs] */
  int32_t* next_free_position; /* [graphs] */
  int32_t position_capacity;
  int32_t chunks_per_graph;
} ckv_delta_chunks;

/* Mutable graph + centroid state (reference: MutableGraphState, graph/state.py:251-349). */
typedef struct ckv_graph_state {
  void* centroids;                   /* [retrieval_heads][community_capacity][128], centroid_dtype */
  int32_t* community_sizes;          /* [retrieval_heads][community_capacity] */
  int32_t* community_counts;         /* [retrieval_heads] */
  float* community_weight;           /* [graph_count][community_capacity] */
  float* total_weight;               /* [graph_count] */
  int32_t* token_communities;        /* [graph_count][token_capacity] */
  const int32_t* retrieval_to_graph; /* [retrieval_heads] */
  const int32_t* retrieval_to_kv;    /* [retrieval_heads] */
  int32_t* current_position;         /* [graph_count] */
  int64_t token_capacity;
  int32_t retrieval_heads;
  int32_t graph_count;
  int32_t community_capacity;
  int32_t centroid_dtype;            /* CKV_E4M3 or CKV_F32 */
} ckv_graph_state;

/* Per-layer decode configuration (reference: CommunityKVConfig, config.py:33-58,
 * plus this build's selection/window/assignment options). */
typedef struct ckv_decode_config {
  const int32_t* sink_positions; /* [num_sink] device */
  int32_t group_size;            /* query heads per retrieval head, 1..16 */
  int32_t num_sink;
  int32_t token_budget;          /* multiple of 64 (reference semantics) */
  int32_t selection_mode;        /* ckv_selection_mode */
  int32_t topk_communities;      /* CKV_SELECT_TOPK only */
  int32_t max_selected;          /* selected-token slots (budget mode: token_budget-num_sink-include_current) */
  int32_t local_window;          /* recent tokens before the current one, set-union with the selection */
  int32_t include_current;       /* 1: attend the current token (reference) */
  int32_t assignment;            /* ckv_assignment */
  int32_t score_coverage;        /* communities per head scored (<= community_capacity) */
  float softmax_scale;
  float lam;
} ckv_decode_config;

/* Preallocated workspace (reference: CentroidSelectionWorkspace centroid_selection.py:191-327,
 * TritonSegmentedAttentionWorkspace segmented_attention.py:953-1013,
 * OnlineUpdateWorkspace graph/kernels/online_update.py:10-35). */
typedef struct ckv_decode_workspace {
  uint16_t* scores;            /* [retrieval_heads][community_capacity] fp16 bits */
  int32_t* communities;        /* [retrieval_heads][descriptor_capacity] */
  int32_t* cumulative_ends;    /* [retrieval_heads][descriptor_capacity] */
  int32_t* descriptor_counts;  /* [retrieval_heads] */
  int32_t* tile_descriptors;   /* [retrieval_heads][budget_tiles] */
  int32_t* selected_counts;    /* [retrieval_heads] */
  int32_t* slot_positions;     /* [retrieval_heads][slot_capacity] KV position per attended slot, -1 = none */
  uint64_t* exchange;          /* [retrieval_heads][community_capacity + 1024], zero before first use, or
                                  null: the fused launch's workgroups of a head hand each other their share of
                                  the centroid scores and nearest-centroid minima through it,
                                  epoch-tagged */
  int32_t* nearest;            /* [retrieval_heads] */
  uint32_t* block_counters;    /* [4 * retrieval_heads], zero before first use: arrival counters (the kernels
                                  leave them zero) and, at [2R, 3R), the fused launch's epoch per head */
  float* partial_max;          /* [query_heads][slot_tiles] */
  float* partial_sum;          /* [query_heads][slot_tiles] */
  float* partial_acc;          /* [query_heads][slot_tiles][128] */
  float* slot_scores;          /* [retrieval_heads][slot_capacity]: scaled score of the group's first query for
                                  every attended slot, the candidates of the update's exact top-8 */
  void* output;                /* [query_heads][128], kv dtype */
  float* lse;                  /* [query_heads] */
  float* topk_scores;          /* [retrieval_heads][8] */
  int32_t* topk_positions;     /* [retrieval_heads][8] */
  int32_t* assigned;           /* [graph_count] */
  int32_t* overflow;           /* [graph_count] bit 1 community, 2 chunk pool, 4 position pool, 8 position */
  int32_t descriptor_capacity;
  int32_t slot_capacity;       /* multiple of 64 */
  int32_t budget_tiles;        /* token_budget / 64 */
  int32_t score_blocks;        /* ceil(score_coverage / 64) */
} ckv_decode_workspace;

/* Causal prefill attention with per-row top-kappa edge export (reference:
 * patched FlashAttention-3 forward, community-kv.patch:31-120, 477-723).
 * bf16 q [S][query_heads][128], k/v [S][kv_heads][128] (row/head strides in
 * elements), GQA head h uses KV head h / (query_heads / kv_heads).
 * Outputs: output like q (bf16), lse [query_heads][S] (natural log of the
 * scaled softmax denominator), and for rows q >= topk_skip the kappa best
 * columns c in [num_sink, q] of row q: topk_indices/topk_scores
 * [query_heads][topk_rows][kappa].  Ranking key: the raw q.k score quantised as
 * clamp(rint((s + 48) * 256), 0, 32767), ties to the larger column (the
 * reference's packed key).  score_kind 0 stores the reference value
 * exp((key/256 - 48) * scale - lse); 1 stores the dequantised raw score
 * key/256 - 48 (within 1/512 of q.k).  seq_len <= 131071. */
typedef struct ckv_prefill_args {
  const void* query;
  const void* key;
  const void* value;
  void* output;
  float* lse;
  float* topk_scores;
  int32_t* topk_indices;
  int64_t q_row_stride;
  int64_t q_head_stride;
  int64_t k_row_stride;
  int64_t k_head_stride;
  int64_t o_row_stride;
  int64_t o_head_stride;
  int32_t seq_len;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t num_sink;
  int32_t kappa;         /* 1..16 */
  int32_t topk_rows;     /* seq_len - topk_skip */
  int32_t topk_skip;     /* num_sink + kappa - 1 */
  int32_t score_kind;    /* 0 probability, 1 dequantised raw score */
  float softmax_scale;
  float reserved;
} ckv_prefill_args;

int ckv_prefill_attention_topk(const ckv_prefill_args* args, void* stream);

/* Prefill graph state from dense community labels (reference: the state build
 * of build_partitioned_layer, graph/partition.py:538-618).
 *
 * ckv_label_counts writes community_counts[g] = 1 + the largest label of graph
 * g's non-sink positions (0 when there are none, -1 when one is negative);
 * the caller reads them back to size the outputs (max_communities = their
 * maximum), as the reference does with .item().
 *
 * ckv_build_layer_state then fills, for labels in [0, max_communities):
 *   member_offsets    [graphs][max_communities + 1]   CSR over non-sink positions
 *   member_positions  [graphs][seq_len - num_sink]    newest first within a community
 *   centroids         [retrieval_heads][community_capacity][128]: mean of the
 *                     community's non-sink keys of KV head retrieval_to_kv[r],
 *                     clamped to +-448, E4M3 or f32; rows past max_communities
 *                     are zero.  The f32 sum runs over the members in
 *                     ascending position order in blocks of 64 (each block
 *                     summed in order, then the block sums in order) and is
 *                     divided by the size
 *   community_sizes   [retrieval_heads][community_capacity]
 *   token_communities [graphs][token_capacity]: the labels, -1 past seq_len
 *   community_weight  [graphs][community_capacity], total_weight [graphs]
 *                     (optional, both or neither): every edge adds its weight
 *                     to both endpoint communities and twice to the total;
 *                     float atomics, so the last bits depend on timing, as
 *                     with the reference's scatter_add_
 * Edge endpoints are graph * seq_len + position.  `workspace` holds
 * ckv_state_workspace_bytes() bytes.  Integer outputs and centroids are
 * deterministic. */
typedef struct ckv_state_build_args {
  const int32_t* labels;              /* [graphs][seq_len] */
  const void* keys;                   /* keys[h*head_stride + t*token_stride + d], key_dtype */
  int64_t head_stride;                /* elements */
  int64_t token_stride;               /* elements */
  const int32_t* retrieval_to_graph;  /* [retrieval_heads] */
  const int32_t* retrieval_to_kv;     /* [retrieval_heads] */
  const int32_t* edge_src;            /* [edges] */
  const int32_t* edge_dst;            /* [edges] */
  const float* edge_weight;           /* [edges] */
  int64_t edges;
  int32_t graphs;
  int32_t seq_len;
  int32_t num_sink;
  int32_t retrieval_heads;
  int32_t kv_heads;
  int32_t key_dtype;                  /* CKV_BF16 or CKV_F32 */
  int32_t centroid_dtype;             /* CKV_E4M3 or CKV_F32 */
  int32_t max_communities;            /* <= CKV_MAX_COMMUNITIES */
  int32_t community_capacity;         /* centroid rows (>= max_communities) */
  int32_t token_capacity;             /* >= seq_len */
  int32_t* member_offsets;
  int32_t* member_positions;
  void* centroids;
  int32_t* community_sizes;
  float* community_weight;            /* may be null (then total_weight too) */
  float* total_weight;
  int32_t* token_communities;
  int32_t* workspace;
  /* Instead of an edge list (then edges == 0): the prefill top-k edges
   * themselves.  Row r of query head h is position topk_row0 + r of graph
   * h / topk_group.  The weights equal those of the reference's
   * build_adjacency (graph/partition.py:168-249: direct edges lam/2 * p,
   * co-occurrence edges (1 - lam) * p_k * p_l for columns k <= l, columns
   * outside [0, seq_len) dropped) followed by init_modularity_state; each row
   * adds its share in closed form, so no edge list is built, sorted or
   * coalesced.  topk_indices == NULL disables this. */
  const int32_t* topk_indices;        /* [topk_heads][topk_rows][topk_kappa] */
  const float* topk_scores;           /* same shape */
  int32_t topk_heads;
  int32_t topk_rows;
  int32_t topk_kappa;                 /* <= 16 */
  int32_t topk_group;                 /* query heads per graph */
  int32_t topk_row0;
  float lam;
} ckv_state_build_args;

size_t ckv_state_workspace_bytes(int32_t graphs, int32_t retrieval_heads, int32_t seq_len, int32_t num_sink,
                                 int32_t max_communities);
int ckv_label_counts(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t num_sink,
                     int32_t* community_counts, void* stream);
int ckv_build_layer_state(const ckv_state_build_args* args, void* stream);

/* One Leiden level over `graphs` vertex-disjoint graphs of seq_len vertices
 * each (vertex ids g * seq_len + i).  Edges: upper-triangular COO (self loops
 * allowed), int32 src/dst, f32 weight, device memory; out-of-range edges are
 * dropped.  Outputs: labels [graphs * seq_len] (a vertex id within the same
 * graph naming the community; -1 for vertices without edges) and
 * modularity [graphs] (f64).  Local moving (up/down gated, up to
 * max_inner_iter sweeps, ends after a stalled sweep in each direction), then
 * refinement inside each local-moving community (greedy, or Gumbel-max at
 * temperature theta when use_boltzmann).  No host synchronisation; workspace
 * of ckv_leiden_workspace_bytes(edges, graphs, seq_len) bytes. */
size_t ckv_leiden_workspace_bytes(int64_t edges, int32_t graphs, int32_t seq_len);
int ckv_batched_leiden(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight, int64_t edges,
                       int32_t graphs, int32_t seq_len, float resolution, float theta, int32_t max_inner_iter,
                       int32_t seed, int32_t use_boltzmann, int32_t* labels, double* modularity,
                       void* workspace, void* stream);

/* Test hook with no counterpart in the reference: while enabled, every
 * ckv_batched_leiden call raises its table-overflow word after the
 * local-moving sweeps, as a broken neighbour-table bound would, so a test can
 * check that the flag survives refinement and turns the level's modularity
 * into NaN (run_leiden then raises).  Process-wide, not thread-safe. */
void ckv_leiden_test_raise_overflow(int32_t enable);

/* Contract an upper-triangular COO by `labels` (super-vertex per vertex, in
 * [0, super_vertices)): both ends relabelled, (min, max) order, duplicates
 * summed, sorted by (src, dst).  Outputs have room for `edges` entries;
 * *out_count (device int64) receives the number written. */
size_t ckv_aggregate_coo_workspace_bytes(int64_t edges);
int ckv_aggregate_coo(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight, int64_t edges,
                      const int32_t* labels, int32_t super_vertices, int32_t* out_src, int32_t* out_dst,
                      float* out_weight, int64_t* out_count, void* workspace, void* stream);

/* The coalesced top-k graph of build_adjacency() (graph/partition.py:168-249):
 * topk_indices / topk_scores [graphs][rows][kappa] (int32 / f32), row r of
 * graph g at position query_positions[g][r] (int64).  Direct edges
 * (position, column) weigh score * lam / 2; when lam < 1, every pair i <= j
 * of a row's columns adds score_i * score_j * (1 - lam).  Columns outside
 * [0, seq_len) are dropped.  Output: upper-triangular COO over global ids
 * g * seq_len + i, sorted by (src, dst), equal pairs summed; room for
 * ckv_adjacency_capacity() entries, *out_count (device int64) = entries
 * written. */
size_t ckv_adjacency_workspace_bytes(int32_t graphs, int32_t rows, int32_t kappa, float lam);
int64_t ckv_adjacency_capacity(int32_t graphs, int32_t rows, int32_t kappa, float lam);
int ckv_build_adjacency(const int32_t* topk_indices, const float* topk_scores, const int64_t* query_positions,
                        int32_t graphs, int32_t rows, int32_t kappa, int32_t seq_len, float lam, int32_t* out_src,
                        int32_t* out_dst, float* out_weight, int64_t* out_count, void* workspace, void* stream);

/* Newman modularity of a labelled edge list taken as one graph (the disjoint
 * union of the per-graph edge lists), labels in [0, vertices): sum of the
 * weights inside communities over m minus resolution * sum of squared
 * community degrees over (2m)^2 (graph/leiden/algorithm.py:166-199, the
 * final modularity of run_leiden()).  *modularity is device f64. */
size_t ckv_partition_modularity_workspace_bytes(int32_t vertices);
int ckv_partition_modularity(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight,
                             int64_t edges, const int32_t* labels, int32_t vertices, float resolution,
                             double* modularity, void* workspace, void* stream);

/* Per-graph dense relabelling: a vertex's label (its own id when negative)
 * becomes its rank among the distinct labels of its graph, plus
 * g * new_seq_len.  ckv_densify_count writes the distinct count per graph
 * (device int32 [graphs]); ckv_densify_apply, with the same workspace and
 * new_seq_len >= every count, writes the dense labels. */
size_t ckv_densify_workspace_bytes(int32_t graphs, int32_t seq_len);
int ckv_densify_count(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t* counts, void* workspace,
                      void* stream);
int ckv_densify_apply(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t new_seq_len, int32_t* dense,
                      const void* workspace, void* stream);

/* Score every retrieval head's centroids against its query group, select the
 * communities that fill the budget (reference order: strictly-above-threshold
 * communities by id, then threshold communities by id, last one truncated),
 * emit descriptors, tile starts and the attended KV position of every slot.
 * With CKV_ASSIGN_NEAREST also finds the current key's nearest centroid. */
int ckv_score_select(const ckv_kv_cache* kv, const ckv_graph_state* state,
                     const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                     const ckv_decode_config* config, ckv_decode_workspace* ws,
                     void* stream);

/* Exact online-softmax attention over the slots chosen by ckv_score_select:
 * split partials, top-8 candidates per split, and the merged output and lse. */
int ckv_segmented_attention(const ckv_kv_cache* kv, const ckv_graph_state* state,
                            const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                            const ckv_decode_config* config, ckv_decode_workspace* ws,
                            void* stream);

/* Diagnostic, no counterpart in the reference: only the split-partials kernel
 * of ckv_segmented_attention, for per-kernel timing and profiling. */
int ckv_attention_partials(const ckv_kv_cache* kv, const ckv_graph_state* state,
                           const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                           const ckv_decode_config* config, ckv_decode_workspace* ws,
                           void* stream);

/* Online update after ckv_segmented_attention (no-op for CKV_ASSIGN_NONE):
 * exact top-8 merge of the splits' candidates, delta-Q or nearest-centroid
 * assignment, running-mean FP8 centroid, decode-delta append, overflow flags,
 * and the layer-wise shared-graph sync.  It may run on a different stream
 * than the next layer's work; it must complete before this layer's next
 * ckv_score_select. */
int ckv_online_update(const ckv_kv_cache* kv, const ckv_graph_state* state,
                      const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                      const ckv_decode_config* config, ckv_decode_workspace* ws,
                      void* stream);

/* The six argument blocks of one layer's decode call. */
typedef struct ckv_layer_args {
  const ckv_kv_cache* kv;
  const ckv_graph_state* state;
  const ckv_prefill_csr* csr;
  const ckv_delta_chunks* deltas;
  const ckv_decode_config* config;
  ckv_decode_workspace* ws;
} ckv_layer_args;

/* Scheduling variant, no counterpart in the reference (whose update is fused
 * into its attention kernel): ckv_score_select of `layer` and, in the same
 * launch on otherwise idle compute units, the deferred ckv_online_update of
 * another layer `pending` (null: none), whose ckv_segmented_attention has
 * already run on this stream.  The two layers' state must be disjoint.  A
 * runtime that defers each layer's update to the next layer's selection takes
 * the update off the decode critical path; it flushes the last one with
 * ckv_online_update. */
int ckv_score_select_after_update(const ckv_layer_args* layer, const ckv_layer_args* pending, void* stream);

/* Batched decode, no counterpart in the reference (whose runtime decodes one
 * sequence at a time; it replaces a loop of decode_layer calls, decode.py:67-111,
 * over independent items): one decode step of `count` items -- the sequences of
 * a ragged batch, or layers whose queries are all ready -- as one selection
 * launch, one attention launch, one split-merge launch and one update launch
 * covering all items, instead of `count` launches of each.  Items must use bf16
 * KV, share the centroid dtype, group size (group_size * 128 <= 512),
 * retrieval-head count, slot capacity and assignment mode, and must not share
 * state or workspace.  `table` is caller-owned device memory of
 * ckv_batch_table_bytes(count) bytes; ckv_batch_prepare validates the items and
 * copies their packed arguments into it, synchronising `stream` (a set-up call:
 * the items' tensors sit at fixed addresses, so one table serves every step).
 * ckv_batch_decode validates the host items again, allocates nothing and does
 * not synchronise; results are identical to ckv_decode_layer on each item.
 * Items may score up to 65536 communities per head; when one item scores more
 * than 8192 the whole batch takes the multi-kernel selection (scoring on
 * every compute unit, 1,024 threads per head) and the separate attention, so
 * an item that alone would take the fused launch gets the same selection and
 * outputs equal up to the order of the split-partial sums. */
size_t ckv_batch_table_bytes(int32_t count);
int ckv_batch_prepare(const ckv_layer_args* items, int32_t count, void* table, void* stream);
int ckv_batch_decode(const ckv_layer_args* items, int32_t count, const void* table, void* stream);
/* Scheduling variant of ckv_batch_decode, no counterpart in the reference
 * (whose update is fused into its attention kernel): one step of `items`
 * whose online update is left pending (the step ends with the split merge),
 * and, on otherwise idle compute units of its selection launch, the pending
 * update of another batch `pending` (null: none; `pending_count` items,
 * `pending_table` prepared by ckv_batch_prepare) whose step has already run on
 * this stream -- the previous layer's batch, so the update leaves the critical
 * path as it does for ckv_decode_step_after_update.  Where the batch takes
 * the fused or the multi-kernel selection the pending update runs in a launch
 * of its own before the step.  The two batches must not share state or
 * workspace.  ckv_batch_online_update runs a batch's pending update by itself
 * (the flush after the last layer).  Results equal ckv_batch_decode's. */
int ckv_batch_decode_after_update(const ckv_layer_args* items, int32_t count, const void* table,
                                  const ckv_layer_args* pending, int32_t pending_count, const void* pending_table,
                                  void* stream);
int ckv_batch_online_update(const ckv_layer_args* items, int32_t count, const void* table, void* stream);
/* (diagnostics) the attention launch of ckv_batch_decode alone, writing split partials. */
int ckv_batch_attention_partials(const ckv_layer_args* items, int32_t count, const void* table, void* stream);

/* Scheduling variant, no counterpart in the reference: one layer's decode
 * (selection + attention; its own online update is left pending) with, in the
 * same launches, the deferred ckv_online_update of another layer `pending`
 * (null: none).  Where the slot table fits in LDS (bf16 KV, at most 8192
 * slots, group_size * 128 <= 512) the selection and the attention partials
 * run in one launch: each retrieval head's slot table is split over several
 * workgroups that each repeat the (latency-bound) selection and attend their
 * own part, so no slot table round-trips through memory and no launch
 * separates selection from attention; a split merge follows.  Otherwise it is
 * ckv_score_select_after_update followed by ckv_segmented_attention. */
int ckv_decode_step_after_update(const ckv_layer_args* layer, const ckv_layer_args* pending, void* stream);
/* (diagnostics) the fused selection + attention-partials launch of
 * ckv_decode_step_after_update alone (no pending update, no merge). */
int ckv_select_attend_partials(const ckv_layer_args* layer, void* stream);

/* ckv_score_select, ckv_segmented_attention and ckv_online_update on one stream. */
int ckv_decode_layer(const ckv_kv_cache* kv, const ckv_graph_state* state,
                     const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                     const ckv_decode_config* config, ckv_decode_workspace* ws,
                     void* stream);

/* Allocation-free variant of ckv_decode_layer, no counterpart in the reference:
 * for callers that cannot allocate device memory (code under graph capture,
 * serving loops that forbid hipMalloc).  The caller passes the state, the KV
 * cache and the outputs (output [query_heads][128] in the kv dtype, lse
 * [query_heads], topk_scores / topk_positions [retrieval_heads][8], assigned /
 * overflow [graph_count]); every other workspace array (scores, descriptors,
 * slot table, exchange row and counters, split partials, per-slot scores)
 * lives in one static device array of ckv_decode_static_scratch_limit() bytes
 * (16 MiB) per GPU, held until the process ends.  Workspace capacities are the
 * ones the Python workspace would allocate for `config` (descriptors
 * min(max_selected or topk_communities, community_capacity), slot capacity
 * ceil((num_sink + max_selected + local_window + include_current) / 64) * 64).
 * A layer needing more scratch than the limit (ckv_decode_static_scratch_bytes)
 * fails with CKV_E_LIMIT.  Calls on one GPU share the array and must not
 * overlap (another stream or host thread): they race.  Each call first runs a
 * one-workgroup kernel that clears the exchange row and counters when the
 * layout stored on the device differs from its own, so eager calls, captured
 * calls and graph replays may follow each other in any order.  Calls no
 * allocator. */
int ckv_decode_layer_static(const ckv_kv_cache* kv, const ckv_graph_state* state,
                            const ckv_prefill_csr* csr, const ckv_delta_chunks* deltas,
                            const ckv_decode_config* config, void* output, float* lse, float* topk_scores,
                            int32_t* topk_positions, int32_t* assigned, int32_t* overflow, void* stream);
size_t ckv_decode_static_scratch_bytes(const ckv_graph_state* state, const ckv_decode_config* config,
                                       int32_t query_heads);
size_t ckv_decode_static_scratch_limit(void);

/* Dense decode baseline: every query head attends positions [0, seq_len) of its
 * KV head (query head h uses KV head h / (query_heads / kv_heads)).  partial_*
 * hold [query_heads][ceil(seq_len/64)] splits. */
int ckv_dense_decode(const ckv_kv_cache* kv, int32_t seq_len, float softmax_scale,
                     float* partial_max, float* partial_sum, float* partial_acc,
                     void* output, float* lse, void* stream);

/* Diagnostic, no counterpart in the reference: latency probes behind the
 * decode step's measured cost model (bench.py --workload floor).  kind 0: one
 * empty kernel of blocks x threads with lds_bytes of dynamic LDS (the host
 * times graphs of them); 1 / 2: `hops` dependent plain / agent-scope loads
 * through the uint32 index cycle in `buffer` (`bytes` long, caller-written);
 * 3: `hops` dependent agent-scope fetch-and-adds on buffer[0]; 4: `hops`
 * hand-offs between two workgroups through buffer[0] (zeroed by the caller,
 * bounded polling); 5: a grid of blocks x threads with lds_bytes of dynamic
 * LDS whose workgroup b writes the id of the XCD it runs on to
 * ((uint32_t*)buffer)[b] (the dispatcher's placement, behind the decode
 * launch's same-XCD score exchange).  Kinds 1-4 write the elapsed 100 MHz
 * wall-clock ticks to out[0] (two device uint64). */
int ckv_latency_probe(int32_t kind, void* buffer, int64_t bytes, int32_t hops, int32_t blocks, int32_t threads,
                      int32_t lds_bytes, uint64_t* out, void* stream);

/* Diagnostic, no counterpart in the reference: evaluates the library's scalar
 * numerics on the host over n inputs, for parity tests without a GPU.
 * op 0 exp -> f32, 1 log -> f32, 2 fp16 bits -> u16, 3 bf16 bits -> u16,
 * 4 E4M3 code -> u8, 5 E4M3 code (given as float) -> f32. */
int ckv_host_numerics(int op, const float* in, void* out, int64_t n);

/* Diagnostic (no reference counterpart): the same ops evaluated by the device
 * functions and gfx950 hardware conversions the kernels use; in/out are device
 * pointers, asynchronous on `stream`. */
int ckv_device_numerics(int op, const float* in, void* out, int64_t n, void* stream);

/* Library version and last error message of the calling thread. */
int ckv_abi_version(void);
const char* ckv_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* CKV_AMD_H */
