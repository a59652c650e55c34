// Internal launch interfaces shared by the kernel files of libpmoe.
#pragma once

#include "pmoe_internal.h"

namespace pmoe {

// Kernel ids of the timing hooks (pmoe_profile_*).
enum KernelId {
  K_ROUTER_LOGITS = 0,
  K_ROUTE_SELECT,
  K_DISPATCH,
  K_GATEUP,
  K_DOWN,
  K_COMBINE,
  K_PREFILL_GATEUP,
  K_PREFILL_DOWN,
  K_DECODE_FUSED,
  K_DECODE_XCD,
  K_EXPERTS_XCD,
  K_COUNT
};

// Brackets the launches in its scope with events when a profile is open.
class ProfScope {
 public:
  ProfScope(int id, hipStream_t st);
  ~ProfScope();

 private:
  int slot_;
  hipStream_t st_;
};

// Component offsets of one projection inside a slab slot.
struct QProj {
  int64_t w, s, b;
};

// Arguments of one grouped dequant-GEMV launch (see decode.hip).
struct GemvArgs {
  const uint8_t* slab;
  int64_t expert_bytes;
  const int32_t* table;  // expert id -> slot (-1: absent)
  int n_experts;         // id n_experts is the shared expert
  int shared_slot;
  QProj p0, p1;          // p1: second projection of a dual (gate/up) launch
  int rows_out;          // output rows of the projection (O)
  int cols;              // input dim
  const uint16_t* act;   // activations, bf16
  int act_stride;        // elements between activation rows
  int act_by_token;      // 1: activation row = flat row / kk; 0: = flat row
  int kk;                // flat columns per token
  const int32_t* active;
  const int32_t* n_active;
  const int32_t* counts;
  const int32_t* offsets;
  const int32_t* order;
  void* out;             // [flat rows, out_stride], f32 or bf16
  int out_stride;
  int out_f32;
};

struct RouteDev;

int qgemv(const GemvArgs& a, int bits, bool dual, int max_experts, int max_rows_per_expert,
          hipStream_t st);
// Router inputs of a decode call (as router_logits_ext takes them; logits
// into out) and the counter the router blocks of a several-token call
// arrive at (kRouteArriveOffset in the workspace header; zero between calls).
struct RouterIn {
  const uint16_t* x;
  const uint16_t* w;
  const uint16_t* w_extra;
  const float* bias;
  int d;
  float* out;
  uint32_t* arrive;
};

// Decode experts (decode.hip): the router launch (which also routes when
// there are several tokens), gate/up, down.  One token: every block
// recomputes the routing.  record: scratch for the routing handed to the
// later launches (decode_record_bytes()).  dn.out: fp32 [n*kk, hidden]
// scratch for the expert-split down (many active experts), or null for the
// tile-major down only.
int decode_routed(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                  int32_t* inds_out, float* w_out, uint16_t* out, void* record,
                  const RouterIn& ri, hipStream_t st);
size_t decode_record_bytes();
// The router launch alone, for any token count (its last block routes and
// writes inds_out / w_out and the record).
int decode_route(const GemvArgs& gu, const RouteDev& rt, int32_t* inds_out, float* w_out,
                 void* record, const RouterIn& ri, hipStream_t st);

// Grid-barrier state of the fused decode launch: the first kDecodeSyncBytes
// of the MoE workspace, zero before the first call.  Blocks arrive in groups
// of kDecodeGroup: group g's counter for barrier i (its own 128-byte line at
// kDecodeGroupOffset + (i * kDecodeMaxGroups + g) * 128) counts the group's
// blocks, and arrive[i] counts the groups that have fully arrived (each
// last arriver resets the counter it completed); epoch counts launches;
// flag line b (128 bytes apart from offset 256) is where block b waits.
struct DecodeSync {
  uint32_t arrive[2];  // groups arrived at barrier 1 / barrier 2
  uint32_t epoch;      // launches completed on this workspace
  uint32_t error;      // sticky: bit 0 = a barrier or data wait timed out,
                       // bit 1 = an expert-per-XCD block group spanned two XCDs
};
// Router blocks of a several-token decode call arrive here (decode.hip
// router_route_kernel; its own 128-byte line; the last arriver resets it).
constexpr size_t kRouteArriveOffset = 128;
constexpr int kDecodeMaxBlocks = 512;
constexpr int kDecodeGroup = 16;  // blocks per arrival group
constexpr int kDecodeMaxGroups = kDecodeMaxBlocks / kDecodeGroup;
constexpr size_t kDecodeFlagStride = 128;  // bytes between two blocks' flags
constexpr size_t kDecodeGroupOffset = 256 + kDecodeMaxBlocks * kDecodeFlagStride;
// Expert-per-XCD launch (decode_fused.hip): one launch counter per block
// group (its own 128-byte line; each of the group's blocks adds 1 per
// launch, so counter / blocks-per-group numbers the launch; the line's next
// two words are the group's masks of XCDs seen, one per launch parity, each
// cleared by the group's last arrival of the launch before), one arrival
// counter per down tile (64 bytes apart; 8 arrivals per launch), each
// group's router logits as tagged 64-bit words (launch tag << 32 | fp32
// bits; every group computes all of them), each group's
// h as tagged 32-bit words (tag & 0xFFFF << 16 | bf16), and each group's
// fp32 down partials.  The given-ids form of that launch (experts_xcd)
// keeps its own launch count in word 4 of each group's counter line (each
// block of the group adds 1 per launch) and its XCD masks in words 5-6, and
// its own regions: the shared expert's h and down rows as 64-bit words
// (launch tag << 32 | bf16 or fp32 bits; every group writes its share, the
// groups read them all), each group's h as tagged 32-bit words and each
// group's fp32 down rows.  Counters only grow and tags name the launch, so
// nothing else is cleared between launches.
constexpr int kXcdCount = 8;
constexpr int kXcdMaxHidden = 8192;
constexpr int kXcdMaxInter = 8192;
constexpr int kXcdMaxTiles = 1024;
constexpr size_t kXcdTileStride = 64;
constexpr size_t kXcdCounterOffset = kDecodeGroupOffset + 2 * kDecodeMaxGroups * kDecodeFlagStride;
constexpr size_t kXcdTileOffset = kXcdCounterOffset + kXcdCount * kDecodeFlagStride;
constexpr size_t kXcdLogitOffset = kXcdTileOffset + kXcdMaxTiles * kXcdTileStride;
constexpr size_t kXcdLogitStride = 512;  // logit words per group (routed experts, at most)
constexpr size_t kXcdHOffset = kXcdLogitOffset + kXcdCount * kXcdLogitStride * sizeof(uint64_t);
constexpr size_t kXcdPartOffset =
    kXcdHOffset + size_t(kXcdCount) * kXcdMaxInter * sizeof(uint32_t);
constexpr int kXcdECounterWord = 4;  // given-ids launch count, then its 2 XCD masks
constexpr size_t kXcdSharedHOffset =
    kXcdPartOffset + size_t(kXcdCount) * kXcdMaxHidden * sizeof(float);
constexpr size_t kXcdSharedPartOffset = kXcdSharedHOffset + size_t(kXcdMaxInter) * sizeof(uint64_t);
constexpr size_t kXcdEHOffset = kXcdSharedPartOffset + size_t(kXcdMaxHidden) * sizeof(uint64_t);
constexpr size_t kXcdEPartOffset =
    kXcdEHOffset + size_t(kXcdCount) * kXcdMaxInter * sizeof(uint32_t);
constexpr size_t kDecodeSyncBytes =
    kXcdEPartOffset + size_t(kXcdCount) * kXcdMaxHidden * sizeof(float);
constexpr int kDecodeFusedDeclined = 1;  // shape not covered: use decode_routed

// Whole decode layer in one persistent launch (decode_fused.hip): router
// logits into rt.logits, routing, gate/up into gu.out (h), down + combine
// into out; one token with top-8 softmax routing and no shared expert takes
// the expert-per-XCD form.  Returns kDecodeFusedDeclined (nothing launched)
// for shapes it does not cover.
int decode_fused(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                 const uint16_t* x, const uint16_t* gate_w, const uint16_t* gate_extra,
                 const float* logit_bias, int32_t* inds_out, float* w_out, uint16_t* out,
                 DecodeSync* sync, hipStream_t st);

// The experts of ONE token given its ids and weights (pmoe_moe_experts'
// arithmetic: each column's output rounded to bf16, combined in column
// order, shared expert last with weight 1, ids outside [0, n_experts) left
// out) in one expert-per-XCD launch: exactly kXcdCount ids, optionally a
// shared expert (no shared gate).  Returns kDecodeFusedDeclined (nothing
// launched) for shapes it does not cover.
// round_y: each column's output rounded to bf16 before the combine
// (pmoe_moe_experts' per-slot outputs); without it the columns combine in
// fp32, as the decode block's expert-split down does.
int experts_xcd(const GemvArgs& gu, const GemvArgs& dn, int bits, int n_experts,
                const int32_t* ids, const float* wts, int shared_slot, uint16_t* out,
                DecodeSync* sync, hipStream_t st, bool round_y = true);
// Whether experts_xcd / the expert-per-XCD form of decode_fused take a shape
// (nothing is launched).
bool experts_xcd_covers(const GemvArgs& gu, const GemvArgs& dn, int bits, int shared_slot);
bool decode_xcd_covers(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                       bool gate_extra);

// Routing (router.hip)
int router_logits(const uint16_t* x, const uint16_t* w, const float* bias, int n, int d, int e,
                  float* out, hipStream_t st);
// Logits [n, e+1]: columns < e from w (+ bias), column e from w_extra.
int router_logits_ext(const uint16_t* x, const uint16_t* w, const uint16_t* w_extra,
                      const float* bias, int n, int d, int e, float* out, hipStream_t st);
int route_softmax(const float* logits, int n, int e, int k, int norm, int32_t* inds,
                  float* weights, hipStream_t st);
int route_sigmoid(const float* logits, const float* bias, int n, int e, int n_group,
                  int topk_group, int k, int norm, float scale, int32_t* inds, float* weights,
                  hipStream_t st);

// Dispatch (dispatch.hip).  Flat row r reads id inds[(r / kk) * k_routed +
// r % kk] when r % kk < k_routed and the shared pseudo-id n_routed otherwise;
// n_ids = n_routed + (kk > k_routed).  With tile_m > 0 it also writes the
// prefill tile list: tile t of id e with c rows is {slot, t * tile_m, c,
// offset of e}, slot = table[e] for routed ids, shared_slot for the shared
// pseudo-id.
size_t dispatch_workspace(int rows, int n_experts);
int dispatch_ext(const int32_t* inds, int rows, int k_routed, int kk, int n_ids,
                 int32_t* order, int32_t* counts, int32_t* offsets, int32_t* inv,
                 int32_t* active, int32_t* n_active, int tile_m, int4* tiles, int32_t* n_tiles,
                 const int32_t* table, int shared_slot, void* ws, size_t ws_bytes,
                 hipStream_t st);

}  // namespace pmoe
