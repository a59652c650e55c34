/* pmoe.h -- C ABI of the MI355X routed-expert MoE hot path (libpmoe.so).
 *
 * Plain pointers and sizes only.  Device pointers are HBM addresses (from
 * hipMalloc, a torch tensor's data_ptr(), or the slab), streams are
 * hipStream_t passed as void* (NULL = the default stream).  Every entry point
 * returns 0 on success and a negative PMOE_E* code on error; the message of
 * the calling thread's last error is pmoe_last_error().  Nothing crosses the
 * ABI as an exception.  Compute entry points allocate nothing: scratch comes
 * in through a caller-provided workspace whose size the *_workspace() query
 * returns.  Calls on one stream are ordered by that stream; calls on
 * different streams that share a workspace race.
 *
 * The reference (noahclark556/paged-moe) has no C ABI for this path: its
 * arithmetic runs inside mlx (gather_qmm / quantized_matmul) called from
 * Python.  Each declaration below names the reference interface it replaces.
 */
#ifndef PMOE_H
#define PMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PMOE_ABI_VERSION 1

enum {
  PMOE_OK = 0,
  PMOE_EINVAL = -1,  /* bad argument or unsupported shape */
  PMOE_EHIP = -2,    /* HIP runtime error */
  PMOE_ENOMEM = -3,  /* allocation failed (create/alloc calls only) */
  PMOE_ESTATE = -4,  /* object in the wrong state */
  PMOE_ESPACE = -5   /* workspace too small */
};

enum { PMOE_SCORE_SOFTMAX = 0, PMOE_SCORE_SIGMOID = 1 };

/* Component order inside one slab slot (names as slab.py:90-126 keys). */
enum {
  PMOE_GATE_W = 0, PMOE_GATE_S, PMOE_GATE_B,
  PMOE_UP_W, PMOE_UP_S, PMOE_UP_B,
  PMOE_DOWN_W, PMOE_DOWN_S, PMOE_DOWN_B,
  PMOE_NCOMP
};

/* Geometry of one quantized SwiGLU expert and its byte layout in a slab
 * slot.  gate/up weight u32 [inter, hidden*bits/32], scales/biases bf16
 * [inter, hidden/group]; down weight u32 [hidden, inter*bits/32],
 * scales/biases bf16 [hidden, inter/group] (safetensors_index.py:8-25,
 * bench/slab_probe.py:82).  off[c] is the byte offset of component c inside a
 * slot, expert_bytes the slot stride. */
typedef struct {
  int32_t hidden;
  int32_t inter;
  int32_t bits;   /* 4 or 6 */
  int32_t group;  /* 64 */
  int64_t expert_bytes;
  int64_t off[PMOE_NCOMP];
  int64_t nbytes[PMOE_NCOMP];
} pmoe_geom;

/* Routing configuration of one MoE block. */
typedef struct {
  int32_t scoring;        /* PMOE_SCORE_* */
  int32_t n_experts;      /* E (routed) */
  int32_t top_k;          /* K */
  int32_t norm_topk_prob; /* renormalise the K weights */
  int32_t n_group;        /* sigmoid: expert groups (1 = none) */
  int32_t topk_group;     /* sigmoid: groups kept */
  float routed_scale;     /* sigmoid: routed_scaling_factor */
} pmoe_route_cfg;

/* ---- library ---------------------------------------------------------- */

/* ABI version of the loaded library (PMOE_ABI_VERSION). No reference
 * counterpart (the reference's native module reports API_VERSION 3,
 * _native_read.c:693, for its read pool only). */
int pmoe_abi_version(void);

/* Last error message of the calling thread ("" if none). */
const char* pmoe_last_error(void);

/* Fill g for an expert of the given shape; the slot layout is
 * component-contiguous in PMOE_* order, each component 256-byte aligned.
 * Replaces SlabStore's per-component specs (slab.py:90-126). */
int pmoe_geom_init(pmoe_geom* g, int hidden, int inter, int bits, int group);

/* ---- routing (replaces mlx-lm's router: gate(x) then softmax/argpartition,
 *      restated tests/test_stream.py:191-196, or deepseek_v3.MoEGate,
 *      consumed streaming.py:2424-2442) ----------------------------------- */

/* logits[n, e] = x[n, :] . w[e, :] (+ logit_bias[e]); x bf16 [n, d], w bf16
 * [e, d], fp32 out, fixed summation order (bit-exact with the CPU oracle).
 * d must be a multiple of 8. */
int pmoe_router_logits(const void* x, const void* w, const float* logit_bias,
                       int n, int d, int e, float* logits, void* stream);

/* Top-k of a softmax router: inds[n, k] (descending weight, ties to the lower
 * expert id) and weights[n, k] fp32. */
int pmoe_route_softmax_topk(const float* logits, int n, int e, int k,
                            int norm_topk_prob, int32_t* inds, float* weights,
                            void* stream);

/* DeepSeek-V3 noaux_tc: sigmoid + bias, grouped top-k, routed scaling. */
int pmoe_route_sigmoid_group_topk(const float* logits, const float* bias,
                                  int n, int e, int n_group, int topk_group,
                                  int k, int norm_topk_prob, float routed_scale,
                                  int32_t* inds, float* weights, void* stream);

/* ---- dispatch (replaces np.argsort(kind="stable") + searchsorted,
 *      streaming.py:789-808, and the unsort inv, :833-836) ---------------- */

size_t pmoe_dispatch_workspace(int rows, int n_experts);

/* Stable grouping of the rows flat positions of inds (int32 [rows]) by
 * expert: order[rows], counts[E], offsets[E+1], inv[rows] (inv[order[i]] =
 * i), active[E] (ascending ids with counts > 0) and *n_active (device). */
int pmoe_dispatch(const int32_t* inds, int rows, int n_experts, int32_t* order,
                  int32_t* counts, int32_t* offsets, int32_t* inv,
                  int32_t* active, int32_t* n_active, void* ws,
                  size_t ws_bytes, void* stream);

/* ---- quantization format (replaces mx.quantize / mx.dequantize semantics
 *      used by QuantizedSwitchLinear; format safetensors_index.py:8-25) ---- */

/* w fp32 [rows, cols] -> q u32 [rows, cols*bits/32], scales/biases bf16
 * [rows, cols/group]; min/max affine, bit-exact with the oracle quantizer. */
int pmoe_quantize(const float* w, int rows, int cols, int bits, int group,
                  uint32_t* q, uint16_t* scales, uint16_t* biases,
                  void* stream);

/* Dequantize to bf16: out = bf16(s*q + b). */
int pmoe_dequant(const uint32_t* q, const uint16_t* scales,
                 const uint16_t* biases, int rows, int cols, int bits,
                 int group, uint16_t* out, void* stream);

/* ---- expert compute --------------------------------------------------- */

/* Workspace bytes for pmoe_switch_glu / pmoe_moe_experts / pmoe_moe_block at
 * n tokens, k routed slots (+ shared: 0 or 1), E experts. */
size_t pmoe_moe_workspace(const pmoe_geom* g, int n, int k, int shared,
                          int n_experts);

/* Rows per tile of the prefill expert GEMMs (the dispatch's row tiles of one
 * expert) for a call of n tokens with kk flat columns per token (top-k plus
 * the shared column) over n_experts routed experts: 32 when the routed
 * experts see at most 32 rows each on average, else 128 (the environment
 * variable PMOE_PREFILL_SMALL=1 / 0 pins 32 / 128).  No reference
 * counterpart (mlx's gather_qmm tiles internally); for callers and tests
 * that reason about tile edges. */
int pmoe_prefill_tile_rows(int n, int kk, int n_experts);

/* A MoE workspace starts with a 1,352,960-byte synchronisation header (grid
 * barrier counters, launch epoch and per-block flags of the one-launch
 * decode layer; launch and tile counters, tagged logit and h words and the
 * down partials of its expert-per-XCD form and of the one-token given-ids
 * pmoe_moe_experts launch; the arrival counter of the
 * several-token decode's router launch, whose last block routes).  It must
 * be zero before the
 * first pmoe_moe_block call on that workspace and is kept consistent by
 * every call after that, so it must not be overwritten between calls.  This
 * enqueues the zeroing on stream (a kernel, so it may be captured in a
 * graph).  No reference counterpart: the reference's decode runs as mlx
 * graph ops with no workspace (streaming.py:587-641). */
int pmoe_moe_workspace_init(void* ws, size_t ws_bytes, void* stream);

/* Synchronising read of the header's sticky error word into *error: bit 0 =
 * a barrier or data wait of the one-launch decode gave up after its spin
 * limit (0.5 s by default); the layer output of that call, and of every later
 * call on the workspace until it is re-initialised, is NaN.  Zeroed only by
 * pmoe_moe_workspace_init. */
int pmoe_moe_workspace_status(const void* ws, uint32_t* error, void* stream);

/* Enqueue on stream a copy of the workspace's error word into host_dst
 * (pinned host memory) without waiting: a caller that synchronises the
 * stream anyway (to read routed ids) reads it after that sync at no extra
 * cost.  No reference counterpart (the reference's mlx graph has no grid
 * barrier that can time out). */
int pmoe_moe_workspace_error_async(const void* ws, uint32_t* host_dst, void* stream);

/* Debug: the one-launch decode's grid-barrier poll limit in 100 MHz
 * realtime-clock ticks (0 restores the default, 0.5 s).  A tiny limit makes
 * every wait give up at once, so tests can check that a timeout poisons the
 * layer output with NaN and sets error bit 0 while every block still exits
 * normally.  Applies to launches issued after the call. */
int pmoe_set_barrier_spin(uint64_t ticks);

/* Debug: with on != 0, block 0 of the expert-per-XCD decode launch reports
 * an XCD other than its own, so its group looks split across two XCDs: the
 * placement check must then set error bit 1 and poison the layer output at
 * once (tests force the failure this way; every block still exits
 * normally).  Applies to launches issued after the call. */
int pmoe_set_split_probe(int on);

/* The seam: y[n, k, :] = FFN_{inds[n,k]}(x[n, :]) as bf16 [n, k, hidden],
 * uncombined, in (token, k) order.  Expert e lives in slab slot table[e]
 * (slab base + slot * expert_bytes).  Replaces
 * StreamedSwitchGLU.__call__(x, indices) (streaming.py:946-1401:
 * _run_slab :587-631 -> three mx.gather_qmm, _gather_proj :504-536). */
int pmoe_switch_glu(const pmoe_geom* g, const void* slab, const int32_t* table,
                    int n_experts, const void* x, const int32_t* inds, int n,
                    int k, void* y, void* ws, size_t ws_bytes, void* stream);

/* Experts + weighted combine given routing: out[n] = sum_k w[n,k] *
 * FFN_{inds[n,k]}(x[n]) (+ shared expert in slot shared_slot, weight 1 or
 * sigmoid(x . shared_gate) when shared_gate != NULL), fp32 accumulation in
 * fixed k order, bf16 out.  shared_slot < 0: no shared expert.  Replaces
 * switch_mlp(x, inds) followed by the block's (y*scores[...,None]).sum(-2)
 * (tests/test_stream.py:198) and the shared-expert add. */
int pmoe_moe_experts(const pmoe_geom* g, const void* slab, const int32_t* table,
                     int n_experts, const void* x, const int32_t* inds,
                     const float* weights, int n, int k, int shared_slot,
                     const void* shared_gate, void* out, void* ws,
                     size_t ws_bytes, void* stream);

/* Whole MoE block: router -> top-k -> dispatch -> experts -> combine.
 * gate_w bf16 [E, hidden]; score_bias fp32 [E] (sigmoid scoring; NULL
 * otherwise); logit_bias fp32 [E] or NULL.  inds_out/weights_out (device,
 * [n, k]) receive the routing.  Replaces the mlx-lm MoE block call around
 * StreamedSwitchGLU: its router (tapped at streaming.py:165-195), top-k,
 * the switch_mlp call (streaming.py:946) and the weighted sum. */
int pmoe_moe_block(const pmoe_geom* g, const pmoe_route_cfg* rc,
                   const void* slab, const int32_t* table, const void* gate_w,
                   const float* score_bias, const float* logit_bias,
                   const void* x, int n, int shared_slot,
                   const void* shared_gate, void* out, int32_t* inds_out,
                   float* weights_out, void* ws, size_t ws_bytes,
                   void* stream);

/* pmoe_moe_block without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static 32 MiB device array of the library, one per GPU,
 * held until the process ends; its address is looked up on the first call
 * on each device, which also zeroes its synchronisation header with a
 * kernel -- so that first call must run outside graph capture (under
 * capture it returns PMOE_ESTATE and launches nothing); later calls may be
 * captured.  Nothing is allocated.  Calls whose workspace would exceed 32 MiB
 * (prefill-sized batches: pmoe_moe_workspace(g, n, k, shared, E) > 32 MiB)
 * return PMOE_ESPACE before anything is launched.  Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (several
 * streams or threads) race; serialise them. */
int pmoe_moe_block_noalloc(const pmoe_geom* g, const pmoe_route_cfg* rc,
                           const void* slab, const int32_t* table,
                           const void* gate_w, const float* score_bias,
                           const float* logit_bias, const void* x, int n,
                           int shared_slot, const void* shared_gate, void* out,
                           int32_t* inds_out, float* weights_out, void* stream);

/* Weighted combine of per-slot outputs: out[n] = bf16(fma over k of
 * weights[n,k] * y[n,k,:], then + s * shared_y[n,:]) with s = 1, or
 * sigmoid(shared_logit[n]) when shared_logit != NULL.  y bf16 [n, k, hidden],
 * shared_y bf16 [n, hidden] or NULL.  The block's
 * (y * scores[..., None]).sum(axis=-2) + shared (tests/test_stream.py:198),
 * used when a layer's experts ran in several fetch groups
 * (cache.py:2535-2578, streaming.py:804-826). */
int pmoe_combine(const void* y, const float* weights, int n, int k, int hidden,
                 const void* shared_y, const float* shared_logit, void* out,
                 void* stream);

/* Closed-stitch miss count (replaces the per-layer miss sum of
 * _closed_forward, streaming.py:905-935, and the token wrapper's one read of
 * it, _closed_call :2843-2870): *counter += the number of ids[0..n) with
 * 0 <= id < n_experts and table[id] < 0, i.e. routed experts the live table
 * does not hold.  One small kernel on stream, no host sync, capturable in a
 * graph; dropped ids (-1) are not counted.  counter is device int32. */
int pmoe_count_missing(const int32_t* table, const int32_t* ids, int n, int n_experts,
                       int32_t* counter, void* stream);

/* ---- slab slot table (replaces ExpertCache's slot policy, cache.py:410:
 *      _alloc_slot :1118-1159, _begin :2327-2453, _finish :2455-2523,
 *      _evict_to_budget :2236-2291, stitch :717-787, flow table :791-859) -- */

typedef struct pmoe_slab pmoe_slab;
typedef struct pmoe_copy_engine pmoe_copy_engine;  /* the copy engine, below */

typedef struct {
  int64_t hits, misses, evictions, starved, installs, resident, slots,
      budget, reserve, stitched, bytes_copied;
  /* prefill fetch groups: misses read into free slots (cache.py:2394-2401
   * prefill_slot_reads), of those installed as resident, misses read into
   * the stage (stage_reads, :1392-1425), misses with neither
   * (prefill_slot_starved + stage_starved), and the stage's size */
  int64_t prefill_slot_reads, prefill_installs, stage_reads, prefill_starved,
      stage_slots;
  /* flow decode: misses admitted (a read started into a slot) */
  int64_t flow_admits;
  /* speculative reads started, claimed by their layer's fetch (of which
   * not yet landed at the claim), and handed back unclaimed */
  int64_t spec_started, spec_claims, spec_claims_late, spec_dropped;
  /* prefill-ahead reads started (prefill_ahead_reads, cache.py:2644) and
   * claimed by the next layer's prefill groups (prefill_ahead_used :2694) */
  int64_t ahead_started, ahead_claims;
} pmoe_slab_stats;

/* Slot policy + device table [n_layers, n_experts] int32 (-1 = absent).
 * The slab memory itself is caller-owned. */
int pmoe_slab_create(pmoe_slab** out, int slots, int n_layers, int n_experts,
                     float reserve_frac, int lfru, int lfru_scan);
int pmoe_slab_destroy(pmoe_slab* s);

/* Device pointer of layer's expert->slot row (n_experts int32). */
const int32_t* pmoe_slab_device_table(pmoe_slab* s, int layer);

/* Host copy of layer's expert->slot row. */
int pmoe_slab_host_table(pmoe_slab* s, int layer, int32_t* out);

/* One layer fetch: ids (host, any order, duplicates allowed) are classified
 * hit/miss, misses get slots (evicting LRU unpinned entries), and are
 * installed in ascending id order with the LFRU second-chance trim.  Writes
 * the misses that got a slot to miss_ids/miss_slots (capacity n_ids) and
 * their count to *n_miss.  Does not touch the GPU. */
int pmoe_slab_request(pmoe_slab* s, int layer, const int32_t* ids, int n_ids,
                      int32_t* miss_ids, int32_t* miss_slots, int* n_miss);

/* Fill every (layer, expert) into fixed slots slot = layer*E + e when they
 * all fit; returns 1 if stitched, 0 if declined. */
int pmoe_slab_stitch(pmoe_slab* s);

/* Enqueue on stream the upload of layer's host table row to the device
 * table. */
int pmoe_slab_publish(pmoe_slab* s, int layer, void* stream);

/* Republish layer's row only if its host copy changed since the last upload
 * (an install, an eviction by any layer's fetch, a prefill group's slots
 * coming back).  Returns 1 if it enqueued an upload, 0 if the row was
 * current, <0 on error.  Replaces flow_table's dirty-row upload
 * (cache.py:843-859, _flow_mark :821-831). */
int pmoe_slab_sync_table(pmoe_slab* s, int layer, void* stream);

/* 1 if layer's device row is stale, 0 if current, <0 on error. */
int pmoe_slab_dirty(pmoe_slab* s, int layer);

/* Inspection: wait for the device, then copy layer's device row (what the
 * kernels read) into out (n_experts int32).  The reference's flow table is
 * an mx.array its caller can read the same way (cache.py:843-859). */
int pmoe_slab_read_device_row(pmoe_slab* s, int layer, int32_t* out);

/* Flow decode's residency update for one layer (flow_admit, cache.py:861-
 * 910): with clear_pins, the pins of the last fetch are dropped first (once
 * per token).  Resident ids get the recency and reuse credit of a fetch hit;
 * other ids are counted as misses and, unless an earlier admit already
 * started their read, take a slot (evicting the least recent entry) and
 * become pending: neither resident nor free, absent from the table, until
 * pmoe_slab_install.  The placed misses go to miss_ids/miss_slots (capacity
 * n_ids).  The caller must know that no queued kernel reads an evicted slot
 * (the reference fences the previous token first) and copies each placed
 * miss into its slot. */
int pmoe_slab_admit(pmoe_slab* s, int layer, const int32_t* ids, int n_ids,
                    int32_t* miss_ids, int32_t* miss_slots, int* n_miss,
                    int clear_pins);

/* Install pending (admitted) experts whose copies have landed: resident at
 * MRU, in the table, with the LFRU trim (the reference's install on arrival,
 * _attach_staging(install_now=True) :2866-2910). */
int pmoe_slab_install(pmoe_slab* s, int layer, const int32_t* ids, int n_ids);

/* The copy engine speculative reads go through (one of its own, so demand
 * copies never queue behind guesses on a stream).  NULL turns speculation
 * off; only allowed while no guess is outstanding. */
int pmoe_slab_set_spec_engine(pmoe_slab* s, pmoe_copy_engine* ce);

/* Prediction-driven prefetch (ExpertCache.prefetch, cache.py:2853, with
 * evict_ok=False): for ids in priority order, skipping resident, pending and
 * already staged ones, take a free slot (never an eviction) while fewer than
 * max_staged guesses are outstanding, and start its read from the host store
 * through the speculation engine, behind that engine's latest fence.
 * *n_started receives the reads started.  A guess is claimed by its layer's
 * pmoe_slab_fetch (or pmoe_slab_request); a fetch hands back that layer's
 * unclaimed guesses, whose slots return once their reads have landed. */
int pmoe_slab_speculate(pmoe_slab* s, const pmoe_geom* g, void* slab,
                        const void* host_store, int layer, const int32_t* ids,
                        int n_ids, int max_staged, int* n_started);

/* Prefill-time prediction (ExpertCache.prefill_ahead, cache.py:2580-2650):
 * a later prefill layer's predicted ids, in priority order, skipping
 * resident, pending and staged ones, take a free routed slot while more than
 * free_floor are free, else a prefill stage slot while more than stage_floor
 * are free (never an eviction), and their reads start through the
 * speculation engine as one copy batch, behind that engine's latest fence.
 * The layer's next pmoe_slab_prefill_request claims the ones it routes (a
 * hit with no new read; the group's row upload joins the batch first) and
 * hands back the rest, whose slots return once the batch has landed.
 * *n_started receives the reads started. */
int pmoe_slab_prefill_ahead(pmoe_slab* s, const pmoe_geom* g, void* slab,
                            const void* host_store, int layer, const int32_t* ids,
                            int n_ids, int free_floor, int stage_floor, int* n_started);

/* Hand back every outstanding guess (flow decode and prefill do not claim
 * them). */
int pmoe_slab_drop_staged(pmoe_slab* s);

/* Register slab slots [first_slot, first_slot + n_slots) (past the routed
 * slots) as the prefill stage: slots prefill misses are read into when no
 * free slot is left, never resident, handed back after each group.
 * Replaces ensure_stage / the stage SlabStore (cache.py:1345-1390). */
int pmoe_slab_set_stage(pmoe_slab* s, int first_slot, int n_slots);

/* Free routed slots, free stage slots, and resident entries the budget
 * still has room for (each may be NULL). */
int pmoe_slab_capacity(pmoe_slab* s, int* free_slots, int* stage_free,
                       int* budget_room);

/* One prefill fetch group's policy step (_begin with prefill=True,
 * PREFILL_TOUCH=0, PREFILL_SLAB=1, cache.py:2347-2453, then
 * _install(..., "soft") :2306-2312): hits keep their recency and frequency;
 * misses, in ascending id, take a free routed slot (never an eviction) and
 * are installed as resident while the resident count is under the budget,
 * else held by this group only; misses past the free slots take stage slots;
 * misses past both are counted in *n_unplaced and get no slot.  The placed
 * misses go to miss_ids/miss_slots (capacity n_ids), their count to *n_miss.
 * *ticket names the group's held slots until pmoe_slab_prefill_done. */
int pmoe_slab_prefill_request(pmoe_slab* s, int layer, const int32_t* ids,
                              int n_ids, int32_t* miss_ids, int32_t* miss_slots,
                              int* n_miss, int* n_unplaced, int* ticket);

/* Enqueue the upload of the group's compute row: the layer's resident
 * entries plus the slots the group holds. */
int pmoe_slab_prefill_publish(pmoe_slab* s, int ticket, void* stream);

/* The group's compute is enqueued: its held free-list and stage slots go
 * back (_release_slot :1101-1116, _stage_return :1427-1440) and the layer's
 * row is marked dirty.  Copies into those slots must be ordered after that
 * compute by a fence (pmoe_copy_fence). */
int pmoe_slab_prefill_done(pmoe_slab* s, int ticket);

int pmoe_slab_stats_get(pmoe_slab* s, pmoe_slab_stats* out);

/* ---- copy engine (replaces the native pread pool, _native_read.c:38-698:
 *      urgent/normal queues, split pieces, promote, first-error latch) ----- */

/* Pinned host memory (hipHostMalloc) for the host expert store. */
int pmoe_host_alloc(void** out, size_t bytes);
int pmoe_host_free(void* p);

/* Engine with its own copy streams (default priority) on the current
 * device; copies are split into pieces of at most split_bytes. */
int pmoe_copy_engine_create(pmoe_copy_engine** out, size_t split_bytes,
                            int n_streams);
int pmoe_copy_engine_destroy(pmoe_copy_engine* ce);

/* Queue a host->device copy; urgent jobs are issued before queued normal
 * ones at the next pmoe_copy_flush. */
int pmoe_copy_submit(pmoe_copy_engine* ce, void* dst, const void* src,
                     size_t bytes, int urgent);

/* Issue every queued job (urgent first) and make stream wait for all of
 * them (event wait, no host block); the copies first wait for everything
 * already queued on stream.  Equals fence(stream) + issue + join(stream). */
int pmoe_copy_flush(pmoe_copy_engine* ce, void* stream);

/* Record the engine's fence on stream: copies issued after this wait for
 * everything queued on stream up to here (a slot is never overwritten while
 * a kernel queued before the fence may read it). */
int pmoe_copy_fence(pmoe_copy_engine* ce, void* stream);

/* Issue every queued job behind the latest fence, without making any
 * stream wait for them (prefill group i+1's reads run under group i's
 * compute, cache.py:2535-2578).  With batch non-NULL the issued copies also
 * form a batch whose completion can be queried, joined and released below
 * (flow decode installs an admitted expert once its read has landed). */
int pmoe_copy_issue(pmoe_copy_engine* ce, int* batch);

/* 1 when every copy of the batch has completed, 0 if not yet, <0 on error. */
int pmoe_copy_batch_done(pmoe_copy_engine* ce, int batch);

/* Make stream wait for the batch's copies. */
int pmoe_copy_batch_join(pmoe_copy_engine* ce, int batch, void* stream);

/* Block the host until the batch's copies have completed. */
int pmoe_copy_batch_wait(pmoe_copy_engine* ce, int batch);

/* Return the batch record (its copies need not have completed). */
int pmoe_copy_batch_release(pmoe_copy_engine* ce, int batch);

/* Make stream wait for every copy issued so far. */
int pmoe_copy_join(pmoe_copy_engine* ce, void* stream);

/* Block until every issued copy has finished; returns the first error. */
int pmoe_copy_sync(pmoe_copy_engine* ce);

/* Bytes issued so far. */
int64_t pmoe_copy_bytes(pmoe_copy_engine* ce);

/* One decode-layer fetch through slab + engine: request(ids), copy each miss
 * from host_store + (layer*n_experts + e)*g->expert_bytes into
 * slab + slot*g->expert_bytes, publish the table on stream and make stream
 * wait for the copies.  *n_miss receives the number of misses copied.
 * Replaces ExpertCache.fetch (cache.py:2525) on the slab path. */
int pmoe_slab_fetch(pmoe_slab* s, pmoe_copy_engine* ce, const pmoe_geom* g,
                    void* slab, const void* host_store, int layer,
                    const int32_t* ids, int n_ids, int* n_miss, void* stream);

/* One prefill fetch group through slab + engine: pmoe_slab_prefill_request,
 * then each placed miss queued from the host store and issued behind the
 * engine's latest fence (pmoe_copy_issue).  Nothing waits for the copies:
 * before the group computes, the caller publishes its row
 * (pmoe_slab_prefill_publish) and joins the copies (pmoe_copy_join).
 * Replaces fetch_groups' per-group _begin(prefill=True) (cache.py:2535-2578). */
int pmoe_slab_fetch_prefill(pmoe_slab* s, pmoe_copy_engine* ce,
                            const pmoe_geom* g, void* slab,
                            const void* host_store, int layer,
                            const int32_t* ids, int n_ids, int* n_miss,
                            int* n_unplaced, int* ticket);

/* ---- slot-safety ledger (replaces PAGED_MOE_SLAB_VERIFY's per-slot
 *      write-in-flight counters and check_slots, cache.py:554-556,
 *      :1171-1206) ----------------------------------------------------------
 * A debug log of every event that orders slot writes against compute: the
 * copy engines record fences, queued copies (dst, src, bytes), issues,
 * joins and host-observed completions; the slab records each row it
 * publishes (a PUBLISH, then one ROW per resident expert); the caller notes
 * each compute it enqueues (pmoe_ledger_note with PMOE_LEDGER_COMPUTE).
 * Off by default; when off nothing is recorded.  One log for the process,
 * in call order; `who` is the engine or slab handle.  A checker replays it
 * and flags a copy issued while an earlier compute may still read its slot,
 * a compute reading a slot whose copy it did not wait for, and a row that
 * maps an expert to a slot holding another. */
enum {
  PMOE_LEDGER_FENCE = 1,      /* who=engine */
  PMOE_LEDGER_SUBMIT = 2,     /* who=engine, a=dst, b=src, c=bytes */
  PMOE_LEDGER_ISSUE = 3,      /* who=engine, a=batch (-1: none) */
  PMOE_LEDGER_JOIN = 4,       /* who=engine: stream waits for every issued copy */
  PMOE_LEDGER_BATCH_JOIN = 5, /* who=engine, a=batch */
  PMOE_LEDGER_HOST_DONE = 6,  /* who=engine, a=batch: the host saw it complete */
  PMOE_LEDGER_HOST_SYNC = 7,  /* who=engine: the host waited for every copy */
  PMOE_LEDGER_PUBLISH = 8,    /* who=slab, a=layer: the row below replaces it */
  PMOE_LEDGER_ROW = 9,        /* who=slab, a=layer, b=expert, c=slot */
  PMOE_LEDGER_COMPUTE = 10    /* who=slab, a=layer: a compute reading the row */
};

typedef struct {
  int64_t kind, who, a, b, c;
} pmoe_ledger_rec;

/* Turn recording on (clearing the log) or off. */
int pmoe_ledger_enable(int on);
/* Append a caller event (PMOE_LEDGER_COMPUTE); ignored while off. */
int pmoe_ledger_note(int64_t kind, const void* who, int64_t a, int64_t b, int64_t c);
/* Move up to cap records, oldest first, into out; *n receives the count.
 * Returns the number of records dropped because the log was full (0). */
int pmoe_ledger_drain(pmoe_ledger_rec* out, int cap, int* n);

/* ---- measurement probes ---------------------------------------------------
 * No reference counterpart.  Kernels of known HBM traffic that bench.py runs
 * next to the kernels it measures: a streaming read with the expert
 * stream's access pattern (16-byte non-temporal loads, 1 KB per wave
 * instruction; the read ceiling), and a 16-byte copy (counter calibration:
 * its FETCH_SIZE / WRITE_SIZE against the bytes it moves). */

/* Bytes of the per-thread sink pmoe_probe_read writes (0 without a device). */
size_t pmoe_probe_sink_bytes(void);

/* Read `bytes` (a multiple of 16, 16-byte aligned) from src; sink receives
 * one xor word per thread. */
int pmoe_probe_read(const void* src, size_t bytes, void* sink, size_t sink_bytes,
                    void* stream);

/* Copy `bytes` (a multiple of 16, both 16-byte aligned) from src to dst. */
int pmoe_probe_copy(void* dst, const void* src, size_t bytes, void* stream);

/* ---- kernel timing --------------------------------------------------------
 * No reference counterpart (the reference splits a token's wall time with
 * host-side wrappers, bench/decode_profile.py).  While a profile is open,
 * every kernel launch of the library is bracketed by HIP events on its own
 * stream; pmoe_profile_end synchronises them and accumulates per-kernel time.
 * Kernel ids are 0..pmoe_profile_kernels()-1. */
int pmoe_profile_begin(int capacity);
int pmoe_profile_end(void);
int pmoe_profile_kernels(void);
const char* pmoe_profile_name(int kernel);
int pmoe_profile_read(int kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* PMOE_H */
