// C-ABI of libmstar_moe: plain pointers, sizes and a stream handle.
//
// Rules for every entry point: the caller owns all buffers (device memory,
// already allocated); nothing here allocates or synchronises; work is
// enqueued on the stream passed in (NULL = the default stream of the current
// device); the return value is 0 or a status code, and
// mstar_moe_last_error() describes the last failure of the calling thread.
// The declarations, with the reference interface each one replaces, are in
// include/mstar_moe.h.
#include <stdarg.h>
#include <stdio.h>

#include <stdlib.h>

#include "common.h"
#include "launch.h"
#include "../../include/mstar_moe.h"

namespace mstar {

static thread_local char g_last_error[512] = "";

void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return kLaunchError;
  }
  return kOk;
}

static size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// Row block for the tiled grouped GEMM: about one block per expert's share of
// the slots, so padding stays a small fraction of the work.  FP8 goes to the
// persistent 256-row kernel from 24 slots per expert on average: despite the
// padding it matches the 32/64-row tiles at 512 and 1024 tokens (E=128, top-8)
// and beats them at 2048 (gate_up + down 177 against 242 us), because the
// one-tile-per-workgroup kernel spends most of the down GEMM's 6 K-steps
// filling its pipeline, and its gate_up epilogue quantises in place.
static int choose_bm(int64_t slots, int E, bool fp8) {
  const int64_t avg = slots / (E > 0 ? E : 1);
  if (fp8 && avg >= 24) return kBigBlockM;
  if (avg <= 48) return 32;
  if (avg <= 160) return 64;
  return 128;
}

// 128-row FP8 tiles below this many slots per expert on average (set from
// the prefill layer's times at E=128, top-8, M = 512 .. 8192).
#ifndef MSTAR_BIG_HALF_MAX_AVG
#define MSTAR_BIG_HALF_MAX_AVG 128
#endif
constexpr int kBigHalfMaxAvg = MSTAR_BIG_HALF_MAX_AVG;

// Largest token count served by the weight-streaming kernels.
constexpr int64_t kStreamMaxTokens = 64;

struct Plan {
  bool stream = false;
  // FP8 weight streaming with the slot lists built inside the GEMMs from the
  // router ids: no alignment launch.
  bool ids_mode = false;
  // The routing launch also quantises the hidden rows (hq/hs in the
  // workspace) for the streaming gate_up GEMM.
  bool route_quant = false;
  // 256-row FP8 GEMMs: the intermediates (FP8 activation codes and, when
  // reduced, the down output) are stored by sorted position, so every tile
  // reads and writes contiguous rows; the top-k sum gathers through pos_of.
  bool by_pos = false;
  // Decode layer (FP8 or W4A16): gate_up and down in one streaming launch
  // (launch_stream_layer), synchronised per expert through off_sync,
  // which the routing launch clears.
  bool one_launch = false;
  // W4A16 above decode size: the 64-token int4 tile GEMM (gemm_w4.hip).
  bool w4_tile = false;
  // FP8 on the persistent tile GEMM (gemm_fp8.hip), bm = 256 or 128 rows.
  bool big = false;
  int bm = 16;
  int64_t slots = 0, max_padded = 0, max_blocks = 0;
  size_t off_sorted, off_eids, off_ntpp, off_eoff, off_ecnt, off_c2, off_c3, off_hq, off_hs,
      off_cq, off_cs, off_scratch, scratch_bytes, off_tw, off_ids, off_pos, off_w4h, off_w4hx, off_w4cx, off_sync, total;
};

// The one-launch decode layer kernel, unless MSTAR_MOE_ONE_LAUNCH=0 in the
// environment (read once).  Its workgroups wait on each other's gate_up
// work but take over whatever is unclaimed before waiting, so concurrent
// launches on one device complete; callers that want no cross-workgroup
// waits at all turn it off and get the two-launch form.
static bool one_launch_enabled() {
  static const bool on = [] {
    const char* v = getenv("MSTAR_MOE_ONE_LAUNCH");
    return !(v && v[0] == '0' && v[1] == 0);
  }();
  return on;
}

// with_route: the plan also holds the router outputs and the routing scratch
// (mstar_moe_layer); otherwise only the alignment scratch (mstar_fused_moe).
static int make_plan(int64_t M, int64_t H, int E, int64_t I, int top_k, int quant, int act_dtype,
                     int reduce, Plan* pl, bool with_route = false) {
  if (M < 0 || H <= 0 || E <= 0 || I <= 0 || top_k <= 0 || top_k > E) {
    set_last_error("fused_moe: invalid sizes (M=%lld H=%lld E=%d I=%lld top_k=%d)",
                   (long long)M, (long long)H, E, (long long)I, top_k);
    return kInvalidArgument;
  }
  if (quant != MSTAR_QUANT_NONE && (H % 128 != 0 || I % 128 != 0)) {
    set_last_error("fused_moe: quantised paths need hidden and intermediate sizes that are "
                   "multiples of 128 (H=%lld I=%lld)", (long long)H, (long long)I);
    return kUnsupported;
  }
  if (quant != MSTAR_QUANT_NONE && act_dtype != kBF16) {
    set_last_error("fused_moe: quantised paths take bf16 activations");
    return kUnsupported;
  }
  if (act_dtype != kBF16 && act_dtype != kF16) {
    set_last_error("fused_moe: activations must be bf16 or fp16");
    return kUnsupported;
  }
  pl->slots = M * top_k;
  const int bkind = quant == MSTAR_QUANT_FP8_W8A8 ? B_FP8BLK : quant == MSTAR_QUANT_W4A16 ? B_INT4G : B_H16;
  pl->stream = quant != MSTAR_QUANT_NONE && M <= kStreamMaxTokens &&
               stream_gemm_supported((int)H, (int)M, A_H16, bkind) &&
               stream_gemm_supported((int)I, (int)M, A_H16, bkind);
  pl->ids_mode = pl->stream && pl->slots <= kStreamMaxIdsSlots &&
                 (quant == MSTAR_QUANT_FP8_W8A8 ||
                  (quant == MSTAR_QUANT_W4A16 && H % 256 == 0 && I % 256 == 0));
  pl->w4_tile = quant == MSTAR_QUANT_W4A16 && !pl->stream && w4_tile_supported(H, I);
  pl->bm = pl->stream ? 16 : pl->w4_tile ? 64 : choose_bm(pl->slots, E, quant == MSTAR_QUANT_FP8_W8A8);
  pl->big = quant == MSTAR_QUANT_FP8_W8A8 && !pl->stream && pl->bm == kBigBlockM;
  // Up to kBigHalfMaxAvg slots per expert on average, 128-row tiles: half the
  // padding per expert and twice the tiles, so the last round of tiles over
  // the CUs wastes less.
  if (pl->big && pl->slots < (int64_t)kBigHalfMaxAvg * E) pl->bm = kBigBlockM / 2;
  pl->max_padded = pl->slots + (int64_t)E * (pl->bm - 1);
  pl->max_blocks = (pl->max_padded + pl->bm - 1) / pl->bm;
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t r = o; o = align_up(o + bytes); return r; };
  pl->off_sorted = take(pl->max_padded * 4);
  pl->off_eids = take(pl->max_blocks * 4);
  pl->off_ntpp = take(4);
  pl->off_eoff = take((size_t)(E + 1) * 4);
  pl->off_ecnt = take((size_t)E * 4);
  const bool fp8_tiled = quant == MSTAR_QUANT_FP8_W8A8 && !pl->stream;
  pl->by_pos = fp8_tiled && pl->big;
  // Rows of the position-indexed buffers: every position of every block.
  const size_t pos_rows = (size_t)pl->max_blocks * pl->bm;
  pl->off_c2 = pl->by_pos ? 0 : take((size_t)pl->slots * I * 2);
  pl->off_c3 = reduce ? take((pl->by_pos ? pos_rows : (size_t)pl->slots) * H * 2) : 0;
  // With the router in the plan, the routing launch quantises the hidden
  // rows: widened to bf16 for the router-ids streaming kernel, as e4m3fn
  // codes for the tiled FP8 GEMM (multi-workgroup routing only).
  pl->route_quant = with_route && ((pl->ids_mode && quant == MSTAR_QUANT_FP8_W8A8 && H % 512 == 0) ||
                                   (quant == MSTAR_QUANT_FP8_W8A8 && !pl->stream &&
                                    route_is_grid(M, top_k)));
  pl->one_launch = one_launch_enabled() && with_route && pl->ids_mode && pl->stream && reduce &&
                   (pl->route_quant || quant == MSTAR_QUANT_W4A16) &&
                   stream_layer_supported(H, I, pl->slots, E, quant == MSTAR_QUANT_W4A16);
  pl->off_sync = pl->one_launch ? take((size_t)layer_sync_words(E, kLayerSyncMaxCus) * 4) : 0;
  pl->off_hq = fp8_tiled ? take((size_t)M * H) : pl->route_quant ? take((size_t)M * H * 2) : 0;
  pl->off_hs = fp8_tiled || pl->route_quant ? take((size_t)M * (H / 128) * 4) : 0;
  const size_t cq_rows = pl->by_pos ? pos_rows : (size_t)pl->slots;
  pl->off_cq = fp8_tiled ? take(cq_rows * I) : 0;
  pl->off_cs = fp8_tiled ? take(cq_rows * (I / 128) * 4) : 0;
  pl->off_pos = pl->by_pos ? take((size_t)pl->slots * 4) : 0;
  // W4 tiles: hidden rows in pair order and their group sums, and the group
  // sums of the gate_up output.
  pl->off_w4h = pl->w4_tile ? take((size_t)M * H * 2) : 0;
  pl->off_w4hx = pl->w4_tile ? take((size_t)M * (H / 128) * 4) : 0;
  pl->off_w4cx = pl->w4_tile ? take((size_t)pl->slots * (I / 128) * 4) : 0;
  pl->scratch_bytes = with_route ? route_scratch_bytes(M, top_k, E) : align_scratch_bytes(pl->slots, E);
  pl->off_scratch = take(pl->scratch_bytes);
  pl->off_tw = with_route ? take((size_t)pl->slots * 4) : 0;
  pl->off_ids = with_route ? take((size_t)pl->slots * 4) : 0;
  pl->total = o;
  return kOk;
}


static int check_layer_args(const Plan& pl, int activation, void* workspace, size_t workspace_bytes) {
  if (activation != 0 && activation != 1) {
    set_last_error("fused_moe: activation must be 0 (silu) or 1 (gelu)");
    return kInvalidArgument;
  }
  if (workspace_bytes < pl.total || (pl.total > 0 && !workspace)) {
    set_last_error("fused_moe: workspace too small (%zu < %zu)", workspace_bytes, pl.total);
    return kWorkspaceTooSmall;
  }
  return kOk;
}

// Everything after the alignment: gate_up GEMM (+ activation), down GEMM
// (x routed weight), top-k sum.  The alignment outputs are in `ws`.
static int run_experts(const Plan& pl, const void* hidden, int act_dtype, int64_t num_tokens,
                       int64_t hidden_size, const void* w1, const void* w2, int num_experts,
                       int64_t inter, int quant, const void* w1_scale, const void* w2_scale,
                       const void* topk_weights, int topk_w_dtype, const void* topk_ids,
                       int ids_dtype, int top_k, int activation, int reduce_results, void* out,
                       uint8_t* ws, hipStream_t stream) {
  const int64_t M = num_tokens, H = hidden_size, I = inter;
  const int E = num_experts;
  int st = kOk;
  int32_t* sorted = (int32_t*)(ws + pl.off_sorted);
  int32_t* eids = (int32_t*)(ws + pl.off_eids);
  int32_t* ntpp = (int32_t*)(ws + pl.off_ntpp);
  int32_t* eoff = (int32_t*)(ws + pl.off_eoff);
  int32_t* ecnt = (int32_t*)(ws + pl.off_ecnt);
  void* cache2 = pl.by_pos ? nullptr : (void*)(ws + pl.off_c2);
  void* cache3 = reduce_results ? (void*)(ws + pl.off_c3) : out;
  const int bkind = quant == MSTAR_QUANT_FP8_W8A8 ? B_FP8BLK : quant == MSTAR_QUANT_W4A16 ? B_INT4G : B_H16;
  GemmArgs g1 = {};
  g1.B = w1;
  g1.C = cache2; g1.ldc = I;
  g1.sorted_ids = sorted; g1.expert_ids = eids; g1.ntpp = ntpp;
  g1.expert_off = eoff; g1.expert_cnt = ecnt;
  g1.M = pl.slots; g1.N = (int)(2 * I); g1.K = (int)H; g1.top_k = top_k; g1.inter = (int)I;
  g1.activation = activation; g1.num_experts = E; g1.m_blocks = (int)pl.max_blocks;
  g1.topk_w = topk_weights; g1.topk_w_dtype = topk_w_dtype;
  if (pl.ids_mode) { g1.topk_ids = topk_ids; g1.ids_dtype = ids_dtype; }
  GemmArgs g2 = g1;
  g2.B = w2;
  g2.C = cache3; g2.ldc = H;
  g2.N = (int)H; g2.K = (int)I; g2.top_k = 1; g2.mul_routed = 1;
  g2.A = cache2; g2.lda = I;

  if (bkind == B_FP8BLK) {
    // w1: [E][2I][H] e4m3fn, scales [E][2I/128][H/128]; w2: [E][H][I], [E][H/128][I/128].
    g1.ldb = H; g1.b_estride = 2 * I * H; g1.b_scale = w1_scale;
    g1.bs_ld = H / 128; g1.bs_estride = (2 * I / 128) * (H / 128);
    g2.ldb = I; g2.b_estride = H * I; g2.b_scale = w2_scale;
    g2.bs_ld = I / 128; g2.bs_estride = (H / 128) * (I / 128);
  } else if (bkind == B_INT4G) {
    // w1: [E][2I][H/8] int32, scales [E][2I][H/128] bf16; w2: [E][H][I/8], [E][H][I/128].
    g1.ldb = H / 8; g1.b_estride = 2 * I * (H / 8); g1.b_scale = w1_scale;
    g1.bs_ld = H / 128; g1.bs_estride = 2 * I * (H / 128);
    g2.ldb = I / 8; g2.b_estride = H * (I / 8); g2.b_scale = w2_scale;
    g2.bs_ld = I / 128; g2.bs_estride = H * (I / 128);
  } else {
    g1.ldb = H; g1.b_estride = 2 * I * H;
    g2.ldb = I; g2.b_estride = H * I;
  }

  if (pl.stream) {
    g1.A = hidden; g1.lda = H;
    if (pl.route_quant) {
      // The routing launch wrote the quantised hidden rows, widened to bf16.
      g1.A = ws + pl.off_hq; g1.a_scale = (const float*)(ws + pl.off_hs); g1.ld_as = H / 128;
      g1.a_q16 = 1;
    }
    if (pl.one_launch) {
      st = launch_stream_layer(g1, g2, bkind == B_INT4G, (int*)(ws + pl.off_sync), stream);
    } else {
      st = launch_stream_gemm(g1, A_H16, bkind, EPI_ACT, act_dtype, (int)M, stream);
      if (st != kOk) return st;
      st = launch_stream_gemm(g2, A_H16, bkind, EPI_STORE, act_dtype, (int)M, stream);
    }
    if (st != kOk) return st;
  } else if (bkind == B_FP8BLK) {
    uint8_t* hq = ws + pl.off_hq;
    float* hs = (float*)(ws + pl.off_hs);
    uint8_t* cq = ws + pl.off_cq;
    float* cs = (float*)(ws + pl.off_cs);
    if (!pl.route_quant) {  // else the routing launch wrote hq / hs
      st = launch_quant_fp8_group(hidden, act_dtype, M, H, H, hq, hs, stream);
      if (st != kOk) return st;
    }
    g1.A = hq; g1.lda = H; g1.a_scale = hs; g1.ld_as = H / 128;
    // The 256-row kernel quantises the activation output in its epilogue;
    // the smaller tiles store bf16 and a quantisation launch follows.
    const bool fused_q = pl.big;
    if (fused_q) { g1.cq = cq; g1.cs = cs; }
    if (pl.by_pos) {
      g1.pos_out = 1;
      g1.pos_of = (int32_t*)(ws + pl.off_pos);
      g2.pos_in = 1;
      g2.pos_out = reduce_results;
    }
    st = pl.big ? launch_gemm_fp8_big(g1, EPI_ACT, true, pl.bm, stream)
                : launch_tile_gemm(g1, A_FP8G, B_FP8BLK, EPI_ACT, act_dtype, true, pl.bm, stream);
    if (st != kOk) return st;
    if (!fused_q) {
      st = launch_quant_fp8_group(cache2, act_dtype, pl.slots, I, I, cq, cs, stream);
      if (st != kOk) return st;
    }
    g2.A = cq; g2.lda = I; g2.a_scale = cs; g2.ld_as = I / 128;
    st = pl.big ? launch_gemm_fp8_big(g2, EPI_STORE, true, pl.bm, stream)
                : launch_tile_gemm(g2, A_FP8G, B_FP8BLK, EPI_STORE, act_dtype, true, pl.bm, stream);
    if (st != kOk) return st;
  } else if (pl.w4_tile) {
    uint16_t* hp = (uint16_t*)(ws + pl.off_w4h);
    float* hx = (float*)(ws + pl.off_w4hx);
    float* cx = (float*)(ws + pl.off_w4cx);
    st = launch_w4_prep(hidden, H, M, H, hp, hx, stream);
    if (st != kOk) return st;
    g1.A = hp; g1.lda = H;
    st = launch_w4_tile(g1, EPI_ACT, hx, cx, stream);
    if (st != kOk) return st;
    st = launch_w4_tile(g2, EPI_STORE, cx, nullptr, stream);
    if (st != kOk) return st;
  } else {
    g1.A = hidden; g1.lda = H;
    st = launch_tile_gemm(g1, A_H16, bkind, EPI_ACT, act_dtype, true, pl.bm, stream);
    if (st != kOk) return st;
    st = launch_tile_gemm(g2, A_H16, bkind, EPI_STORE, act_dtype, true, pl.bm, stream);
    if (st != kOk) return st;
  }
  if (reduce_results && pl.by_pos)
    return launch_sum_reduce_pos(cache3, (const int32_t*)(ws + pl.off_pos), out, act_dtype, M, top_k, H,
                                 stream);
  if (reduce_results)
    return launch_sum_reduce(cache3, out, act_dtype, M, top_k, H, 1.0f, stream);
  return kOk;
}

}  // namespace mstar

using namespace mstar;

extern "C" {

const char* mstar_moe_last_error(void) { return g_last_error; }

int mstar_moe_abi_version(void) { return MSTAR_MOE_ABI_VERSION; }

int mstar_moe_topk_softmax(const void* logits, int logits_dtype, int64_t num_tokens,
                           int num_experts, int top_k, int renormalize, float* topk_weights,
                           int32_t* topk_ids_i32, int64_t* topk_ids_i64, void* stream) {
  return launch_topk_softmax(logits, logits_dtype, num_tokens, num_experts, top_k, renormalize,
                             topk_weights, topk_ids_i32, topk_ids_i64, (hipStream_t)stream);
}

int mstar_moe_router(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                     const void* gate_weight, int num_experts, int top_k, int renormalize,
                     float* topk_weights, int32_t* topk_ids_i32, int64_t* topk_ids_i64,
                     void* logits_out, void* stream) {
  if (act_dtype != kBF16) {
    set_last_error("router: hidden states and gate weight must be bfloat16");
    return kUnsupported;
  }
  return launch_router(hidden, num_tokens, hidden_size, gate_weight, num_experts, top_k, renormalize,
                       topk_weights, topk_ids_i32, topk_ids_i64, logits_out, (hipStream_t)stream);
}

int mstar_moe_topk_softmax_quant(const void* logits, int logits_dtype, int64_t num_tokens,
                                 int num_experts, int top_k, int renormalize,
                                 float* topk_weights, int32_t* topk_ids_i32,
                                 int64_t* topk_ids_i64, const void* hidden, int64_t hidden_size,
                                 void* hidden_q, float* hidden_scale, void* stream) {
  if (!hidden || !hidden_q || !hidden_scale) {
    set_last_error("topk_softmax_quant: null hidden / hidden_q / hidden_scale");
    return kInvalidArgument;
  }
  return launch_topk_softmax(logits, logits_dtype, num_tokens, num_experts, top_k, renormalize,
                             topk_weights, topk_ids_i32, topk_ids_i64, (hipStream_t)stream,
                             hidden, hidden_size, (uint16_t*)hidden_q, hidden_scale);
}

int mstar_moe_stream_gemm(const void* A, int a_dtype, const float* a_scale, const void* B,
                          const float* b_scale, void* C, const void* topk_weights,
                          int topk_w_dtype, const void* topk_ids, int ids_dtype,
                          int64_t num_slots, int num_experts, int64_t N, int64_t K, int top_k,
                          int mul_routed_weight, int activation, void* stream) {
  if (num_slots < 0 || num_slots > kStreamMaxIdsSlots || num_experts <= 0 || N <= 0 || K <= 0 ||
      top_k <= 0 || activation < -1 || activation > 1 || (activation >= 0 && N % 2 != 0)) {
    set_last_error("moe_stream_gemm: invalid sizes (slots=%lld E=%d N=%lld K=%lld top_k=%d)",
                   (long long)num_slots, num_experts, (long long)N, (long long)K, top_k);
    return kInvalidArgument;
  }
  if (a_dtype != kBF16 && a_dtype != MSTAR_DTYPE_FP8_AS_BF16) {
    set_last_error("moe_stream_gemm: A must be bf16 or FP8_AS_BF16");
    return kUnsupported;
  }
  if (ids_dtype != kI32 && ids_dtype != kI64) {
    set_last_error("moe_stream_gemm: topk_ids must be int32 or int64");
    return kUnsupported;
  }
  if (num_slots == 0) return kOk;
  if (!A || !B || !b_scale || !C || !topk_ids || (a_dtype != kBF16 && !a_scale) ||
      (mul_routed_weight && !topk_weights)) {
    set_last_error("moe_stream_gemm: null tensor pointer");
    return kInvalidArgument;
  }
  GemmArgs g = {};
  g.A = A; g.lda = K;
  if (a_dtype != kBF16) { g.a_scale = a_scale; g.ld_as = K / 128; g.a_q16 = 1; }
  g.B = B; g.ldb = K; g.b_estride = N * K; g.b_scale = b_scale;
  g.bs_ld = K / 128; g.bs_estride = ((N + 127) / 128) * (K / 128);
  g.C = C; g.ldc = activation >= 0 ? N / 2 : N;
  g.topk_w = topk_weights; g.topk_w_dtype = topk_w_dtype;
  g.topk_ids = topk_ids; g.ids_dtype = ids_dtype;
  g.M = num_slots; g.N = (int)N; g.K = (int)K; g.top_k = top_k; g.inter = (int)(N / 2);
  g.mul_routed = mul_routed_weight; g.activation = activation < 0 ? 0 : activation;
  g.num_experts = num_experts;
  return launch_stream_fp8(g, activation >= 0 ? EPI_ACT : EPI_STORE, true, (hipStream_t)stream);
}

int mstar_moe_stream_layer(const void* hq, const float* hs, const void* w1, const float* w1_scale,
                           const void* w2, const float* w2_scale, const float* topk_weights,
                           const int32_t* topk_ids, int64_t num_tokens, int64_t hidden,
                           int num_experts, int64_t inter, int top_k, int activation, void* act,
                           void* out_rows, int32_t* sync, void* stream) {
  if (num_tokens < 0 || hidden <= 0 || inter <= 0 || num_experts <= 0 || top_k <= 0 ||
      top_k > num_experts || activation < 0 || activation > 1) {
    set_last_error("moe_stream_layer: invalid sizes (M=%lld H=%lld E=%d I=%lld top_k=%d act=%d)",
                   (long long)num_tokens, (long long)hidden, num_experts, (long long)inter, top_k,
                   activation);
    return kInvalidArgument;
  }
  const int64_t slots = num_tokens * top_k;
  if (!stream_layer_supported(hidden, inter, slots, num_experts, false)) {
    set_last_error("moe_stream_layer: unsupported shape (H=%lld I=%lld slots=%lld E=%d)",
                   (long long)hidden, (long long)inter, (long long)slots, num_experts);
    return kUnsupported;
  }
  if (num_tokens == 0) return kOk;
  if (!hq || !hs || !w1 || !w1_scale || !w2 || !w2_scale || !topk_weights || !topk_ids || !act ||
      !out_rows || !sync) {
    set_last_error("moe_stream_layer: null tensor pointer");
    return kInvalidArgument;
  }
  const int64_t H = hidden, I = inter;
  GemmArgs g1 = {};
  g1.A = hq; g1.lda = H; g1.a_scale = hs; g1.ld_as = H / 128; g1.a_q16 = 1;
  g1.B = w1; g1.ldb = H; g1.b_estride = 2 * I * H; g1.b_scale = w1_scale;
  g1.bs_ld = H / 128; g1.bs_estride = (2 * I / 128) * (H / 128);
  g1.C = act; g1.ldc = I;
  g1.topk_w = topk_weights; g1.topk_w_dtype = kF32;
  g1.topk_ids = topk_ids; g1.ids_dtype = kI32;
  g1.M = slots; g1.N = (int)(2 * I); g1.K = (int)H; g1.top_k = top_k; g1.inter = (int)I;
  g1.activation = activation; g1.num_experts = num_experts;
  GemmArgs g2 = g1;
  g2.A = act; g2.lda = I; g2.a_scale = nullptr; g2.ld_as = 0; g2.a_q16 = 0;
  g2.B = w2; g2.ldb = I; g2.b_estride = H * I; g2.b_scale = w2_scale;
  g2.bs_ld = I / 128; g2.bs_estride = (H / 128) * (I / 128);
  g2.C = out_rows; g2.ldc = H;
  g2.N = (int)H; g2.K = (int)I; g2.top_k = 1; g2.mul_routed = 1;
  return launch_stream_layer(g1, g2, false, sync, (hipStream_t)stream);
}

int mstar_moe_layer_wait_failures(int* count) { return layer_wait_failures(count); }

int mstar_moe_layer_sync_words(int num_experts, int64_t* words) {
  if (num_experts <= 0 || num_experts > 1024 || !words) {
    set_last_error("moe_layer_sync_words: invalid arguments (E=%d)", num_experts);
    return kInvalidArgument;
  }
  *words = layer_sync_words(num_experts, kLayerSyncMaxCus);
  return kOk;
}

int mstar_moe_debug_layer_test_mode(int mode) { return set_layer_test_mode(mode); }

int mstar_moe_align_block_size(const void* topk_ids, int ids_dtype, int64_t numel,
                               int num_experts, int block_size, int32_t* sorted_token_ids,
                               int64_t sorted_len, int32_t* expert_ids, int64_t expert_ids_len,
                               int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                               int32_t* expert_counts, void* scratch, size_t scratch_bytes,
                               void* stream) {
  if (block_size > 0 && expert_ids_len < (sorted_len + block_size - 1) / block_size) {
    set_last_error("moe_align_block_size: experts_ids too small (%lld < %lld)",
                   (long long)expert_ids_len,
                   (long long)((sorted_len + block_size - 1) / block_size));
    return kInvalidArgument;
  }
  return launch_align(topk_ids, ids_dtype, numel, num_experts, block_size, sorted_token_ids,
                      expert_ids, num_tokens_post_pad, sorted_len, expert_offsets, expert_counts,
                      scratch, scratch_bytes, (hipStream_t)stream);
}

int mstar_moe_act_and_mul(const void* gate_up, void* out, int dtype, int64_t rows, int64_t inter,
                          int activation, void* stream) {
  return launch_act_and_mul(gate_up, out, dtype, rows, inter, activation, (hipStream_t)stream);
}

int mstar_moe_sum_reduce(const void* input, void* output, int dtype, int64_t tokens,
                         int64_t top_k, int64_t hidden, float routed_scaling_factor,
                         void* stream) {
  return launch_sum_reduce(input, output, dtype, tokens, top_k, hidden, routed_scaling_factor,
                           (hipStream_t)stream);
}

int mstar_quant_fp8_per_token_group(const void* x, int dtype, int64_t rows, int64_t cols,
                                    int group_size, uint8_t* q, float* scales, void* stream) {
  if (group_size != 128) {
    set_last_error("quant_fp8_per_token_group: only group_size 128 is supported");
    return kUnsupported;
  }
  return launch_quant_fp8_group(x, dtype, rows, cols, cols, q, scales, (hipStream_t)stream);
}

int mstar_quant_fp8_per_token(const void* x, int dtype, int64_t rows, int64_t cols, uint8_t* q,
                              float* scales, void* stream) {
  return launch_quant_fp8_row(x, dtype, rows, cols, q, scales, (hipStream_t)stream);
}

int mstar_fp8_scaled_mm(const uint8_t* a, const float* a_scale, const uint8_t* w,
                        const float* w_scale, void* out, int64_t M, int64_t N, int64_t K,
                        void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || N >= (1ll << 31) || K % 128 != 0 || !out ||
      (M > 0 && (!a || !a_scale || !w || !w_scale))) {
    set_last_error("fp8_scaled_mm: invalid arguments (M=%lld N=%lld K=%lld; K %% 128 == 0)",
                   (long long)M, (long long)N, (long long)K);
    return kInvalidArgument;
  }
  if (M == 0) return kOk;
  GemmArgs g = {};
  g.A = a; g.lda = K; g.a_scale = a_scale;
  g.B = w; g.ldb = K; g.b_estride = 0; g.b_scale = w_scale;
  g.C = out; g.ldc = N;
  g.M = M; g.N = (int)N; g.K = (int)K; g.top_k = 1;
  if (dense_stream_supported(M, N, K)) {
    const int st = launch_dense_stream(g, (hipStream_t)stream);
    if (st != kUnsupported) return st;  // else the tile kernel below
  }
  if (M > 64) {
    // 256-row tiles, or 128-row tiles when the 256-row ones would not give
    // every CU a tile (N=2048 at M=4096: 128 tiles of 256 rows for 256 CUs).
    const int64_t tiles256 = ((M + kBigBlockM - 1) / kBigBlockM) * ((N + 255) / 256);
    const int cus = device_cu_count();
    if (cus <= 0) return kLaunchError;
    const int bm = tiles256 < cus ? kBigBlockM / 2 : kBigBlockM;
    return launch_gemm_fp8_big(g, EPI_DENSE, false, bm, (hipStream_t)stream);
  }
  return launch_tile_gemm(g, A_FP8R, B_FP8R, EPI_DENSE, kBF16, false, M <= 32 ? 32 : 64,
                          (hipStream_t)stream);
}

int mstar_moe_grouped_gemm(const void* A, const void* B, void* C, const void* topk_weights,
                           int topk_w_dtype, const int32_t* sorted_token_ids,
                           const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                           int64_t N, int64_t K, int64_t em, int64_t num_valid_tokens, int top_k,
                           int mul_routed_weight, int block_size, int dtype, void* stream) {
  if (N <= 0 || K <= 0 || em < 0 || top_k <= 0 || !A || !B || !C || !sorted_token_ids ||
      !expert_ids || !num_tokens_post_padded || (mul_routed_weight && !topk_weights)) {
    set_last_error("moe_grouped_gemm: invalid arguments");
    return kInvalidArgument;
  }
  GemmArgs g = {};
  g.A = A; g.lda = K;
  g.B = B; g.ldb = K; g.b_estride = N * K;
  g.C = C; g.ldc = N;
  g.topk_w = topk_weights; g.topk_w_dtype = topk_w_dtype;
  g.sorted_ids = sorted_token_ids; g.expert_ids = expert_ids; g.ntpp = num_tokens_post_padded;
  g.M = num_valid_tokens; g.N = (int)N; g.K = (int)K; g.top_k = top_k;
  g.mul_routed = mul_routed_weight;
  g.m_blocks = (int)((em + block_size - 1) / block_size);
  return launch_tile_gemm(g, A_H16, B_H16, EPI_STORE, dtype, true, block_size,
                          (hipStream_t)stream);
}

int mstar_moe_gemm(const void* A, int a_dtype, const float* a_scale, const void* B, int quant,
                   const void* b_scale, void* C, int c_dtype, const void* topk_weights,
                   int topk_w_dtype, const int32_t* sorted_token_ids, const int32_t* expert_ids,
                   const int32_t* num_tokens_post_padded, const int32_t* expert_offsets,
                   const int32_t* expert_counts, int num_experts, int64_t N, int64_t K,
                   int64_t em, int64_t num_valid_tokens, int top_k, int mul_routed_weight,
                   int activation, int block_size, int path, void* stream) {
  if (N <= 0 || K <= 0 || (quant != MSTAR_QUANT_NONE && K % 128 != 0) || num_experts <= 0 || top_k <= 0 || !A || !B || !C ||
      !sorted_token_ids || (mul_routed_weight && !topk_weights) ||
      (quant != MSTAR_QUANT_NONE && !b_scale) || activation < -1 || activation > 1 ||
      (activation >= 0 && N % 2 != 0) || path < 0 || path > 2) {
    set_last_error("moe_gemm: invalid arguments (N=%lld K=%lld quant=%d act=%d path=%d)",
                   (long long)N, (long long)K, quant, activation, path);
    return kInvalidArgument;
  }
  const int bkind = quant == MSTAR_QUANT_FP8_W8A8 ? B_FP8BLK : quant == MSTAR_QUANT_W4A16 ? B_INT4G : B_H16;
  GemmArgs g = {};
  g.A = A; g.lda = K; g.a_scale = a_scale; g.ld_as = K / 128;
  g.B = B; g.b_scale = b_scale;
  if (bkind == B_FP8BLK) {
    g.ldb = K; g.b_estride = N * K; g.bs_ld = K / 128; g.bs_estride = ((N + 127) / 128) * (K / 128);
  } else if (bkind == B_INT4G) {
    g.ldb = K / 8; g.b_estride = N * (K / 8); g.bs_ld = K / 128; g.bs_estride = N * (K / 128);
  } else {
    g.ldb = K; g.b_estride = N * K;
  }
  g.C = C; g.ldc = activation >= 0 ? N / 2 : N;
  g.topk_w = topk_weights; g.topk_w_dtype = topk_w_dtype;
  g.sorted_ids = sorted_token_ids; g.expert_ids = expert_ids; g.ntpp = num_tokens_post_padded;
  g.expert_off = expert_offsets; g.expert_cnt = expert_counts;
  g.M = num_valid_tokens; g.N = (int)N; g.K = (int)K; g.top_k = top_k;
  g.inter = (int)(N / 2); g.mul_routed = mul_routed_weight;
  g.activation = activation < 0 ? 0 : activation; g.num_experts = num_experts;
  g.m_blocks = block_size > 0 ? (int)((em + block_size - 1) / block_size) : 0;
  const int epi = activation >= 0 ? EPI_ACT : EPI_STORE;
  const bool a16 = a_dtype == kBF16 || a_dtype == kF16;
  if (path == 2 || (path == 0 && a16 && bkind != B_H16 && expert_offsets && expert_counts &&
                    stream_gemm_supported((int)K, 0, A_H16, bkind) &&
                    num_valid_tokens <= 64 * top_k)) {
    if (!a16) {
      set_last_error("moe_gemm: the streaming path takes 16-bit activations");
      return kUnsupported;
    }
    return launch_stream_gemm(g, A_H16, bkind, epi, a_dtype, 0, (hipStream_t)stream);
  }
  if (!expert_ids || !num_tokens_post_padded) {
    set_last_error("moe_gemm: the tiled path needs expert_ids and num_tokens_post_padded");
    return kInvalidArgument;
  }
  int akind = A_H16;
  if (a_dtype == kFP8) {
    if (!a_scale) {
      set_last_error("moe_gemm: FP8 activations need per-128-group scales");
      return kInvalidArgument;
    }
    akind = A_FP8G;
  }
  if ((akind == A_FP8G) != (bkind == B_FP8BLK)) {
    set_last_error("moe_gemm: FP8 weights need FP8 activations on the tiled path");
    return kUnsupported;
  }
  const int dt = a16 ? a_dtype : c_dtype;
  return launch_tile_gemm(g, akind, bkind, epi, dt, true, block_size, (hipStream_t)stream);
}

int mstar_fused_moe_workspace_size(int64_t num_tokens, int64_t hidden, int num_experts,
                                   int64_t inter, int top_k, int quant, int act_dtype,
                                   int reduce_results, size_t* bytes) {
  Plan pl;
  int st = make_plan(num_tokens, hidden, num_experts, inter, top_k, quant, act_dtype,
                     reduce_results, &pl);
  if (st == kOk && bytes) *bytes = pl.total;
  return st;
}

int mstar_fused_moe(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* w1, const void* w2, int num_experts, int64_t inter, int quant,
                    const void* w1_scale, const void* w2_scale, const void* topk_weights,
                    int topk_w_dtype, const void* topk_ids, int ids_dtype, int top_k,
                    int activation, int reduce_results, void* out, void* workspace,
                    size_t workspace_bytes, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  Plan pl;
  int st = make_plan(num_tokens, hidden_size, num_experts, inter, top_k, quant, act_dtype,
                     reduce_results, &pl);
  if (st != kOk) return st;
  if ((st = check_layer_args(pl, activation, workspace, workspace_bytes)) != kOk) return st;
  if (num_tokens == 0) return kOk;
  if (!hidden || !w1 || !w2 || !topk_weights || !topk_ids || !out ||
      (quant != MSTAR_QUANT_NONE && (!w1_scale || !w2_scale))) {
    set_last_error("fused_moe: null tensor pointer");
    return kInvalidArgument;
  }
  if (ids_dtype != kI32 && ids_dtype != kI64) {
    set_last_error("fused_moe: topk_ids must be int32 or int64");
    return kUnsupported;
  }
  uint8_t* ws = (uint8_t*)workspace;
  if (!pl.ids_mode) {
    st = launch_align(topk_ids, ids_dtype, pl.slots, num_experts, pl.bm,
                      (int32_t*)(ws + pl.off_sorted), (int32_t*)(ws + pl.off_eids),
                      (int32_t*)(ws + pl.off_ntpp), pl.max_padded, (int32_t*)(ws + pl.off_eoff),
                      (int32_t*)(ws + pl.off_ecnt), ws + pl.off_scratch, pl.scratch_bytes, stream);
    if (st != kOk) return st;
  }
  return run_experts(pl, hidden, act_dtype, num_tokens, hidden_size, w1, w2, num_experts, inter,
                     quant, w1_scale, w2_scale, topk_weights, topk_w_dtype, topk_ids, ids_dtype,
                     top_k, activation, reduce_results, out, ws, stream);
}

int mstar_moe_layer_workspace_size(int64_t num_tokens, int64_t hidden, int num_experts,
                                   int64_t inter, int top_k, int quant, int act_dtype,
                                   size_t* bytes) {
  Plan pl;
  int st = make_plan(num_tokens, hidden, num_experts, inter, top_k, quant, act_dtype, 1, &pl, true);
  if (st == kOk && bytes) *bytes = pl.total;
  return st;
}

extern "C++" {
namespace mstar {
// mstar_moe_layer; allow_one_launch = false keeps the decode layer in its
// two-launch form (no sync words, no waits between workgroups).
int moe_layer_impl(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                   const void* router_logits, int logits_dtype, int renormalize, const void* w1,
                   const void* w2, int num_experts, int64_t inter, int quant,
                   const void* w1_scale, const void* w2_scale, int top_k, int activation,
                   void* out, float* topk_weights_out, int64_t* topk_ids_out, void* workspace,
                   size_t workspace_bytes, void* stream_, bool allow_one_launch) {
  hipStream_t stream = (hipStream_t)stream_;
  Plan pl;
  int st = make_plan(num_tokens, hidden_size, num_experts, inter, top_k, quant, act_dtype, 1, &pl,
                     true);
  if (st != kOk) return st;
  if (!allow_one_launch) pl.one_launch = false;
  int sync_clear = 0;
  if (pl.one_launch) {
    const int cus = device_cu_count();
    if (cus <= 0) return kLaunchError;
    sync_clear = layer_sync_words(num_experts, cus < kLayerSyncMaxCus ? cus : kLayerSyncMaxCus);
  }
  if ((st = check_layer_args(pl, activation, workspace, workspace_bytes)) != kOk) return st;
  if (num_tokens == 0) return kOk;
  if (!hidden || !router_logits || !w1 || !w2 || !out ||
      (quant != MSTAR_QUANT_NONE && (!w1_scale || !w2_scale))) {
    set_last_error("moe_layer: null tensor pointer");
    return kInvalidArgument;
  }
  uint8_t* ws = (uint8_t*)workspace;
  float* tw = topk_weights_out ? topk_weights_out : (float*)(ws + pl.off_tw);
  int32_t* ids32 = (int32_t*)(ws + pl.off_ids);
  if (pl.ids_mode)
    st = launch_topk_softmax(router_logits, logits_dtype, num_tokens, num_experts, top_k,
                             renormalize, tw, ids32, topk_ids_out, stream,
                             pl.route_quant ? hidden : nullptr, hidden_size,
                             (uint16_t*)(ws + pl.off_hq), (float*)(ws + pl.off_hs),
                             pl.one_launch ? (int*)(ws + pl.off_sync) : nullptr, sync_clear);
  else
    st = launch_route(router_logits, logits_dtype, num_tokens, num_experts, top_k, renormalize, tw,
                      ids32, topk_ids_out, pl.bm, (int32_t*)(ws + pl.off_sorted),
                      (int32_t*)(ws + pl.off_eids), (int32_t*)(ws + pl.off_ntpp), pl.max_padded,
                      (int32_t*)(ws + pl.off_eoff), (int32_t*)(ws + pl.off_ecnt),
                      ws + pl.off_scratch, pl.scratch_bytes, stream,
                      pl.route_quant ? hidden : nullptr, hidden_size, ws + pl.off_hq,
                      (float*)(ws + pl.off_hs));
  if (st != kOk) return st;
  return run_experts(pl, hidden, act_dtype, num_tokens, hidden_size, w1, w2, num_experts, inter,
                     quant, w1_scale, w2_scale, tw, kF32, ids32, kI32, top_k, activation, 1, out,
                     ws, stream);
}
}  // namespace mstar
}  // extern "C++"

int mstar_moe_layer(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* router_logits, int logits_dtype, int renormalize, const void* w1,
                    const void* w2, int num_experts, int64_t inter, int quant,
                    const void* w1_scale, const void* w2_scale, int top_k, int activation,
                    void* out, float* topk_weights_out, int64_t* topk_ids_out, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return moe_layer_impl(hidden, act_dtype, num_tokens, hidden_size, router_logits, logits_dtype,
                        renormalize, w1, w2, num_experts, inter, quant, w1_scale, w2_scale, top_k,
                        activation, out, topk_weights_out, topk_ids_out, workspace, workspace_bytes,
                        stream, true);
}

int mstar_moe_block(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* gate_weight, int renormalize, const void* w1, const void* w2,
                    int num_experts, int64_t inter, int quant, const void* w1_scale,
                    const void* w2_scale, int top_k, int activation, void* out,
                    float* topk_weights_out, int64_t* topk_ids_out, void* logits_out,
                    void* workspace, size_t workspace_bytes, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (act_dtype != kBF16) {
    set_last_error("moe_block: the fused router takes bf16 hidden states and gate weight");
    return kUnsupported;
  }
  Plan pl;
  int st = make_plan(num_tokens, hidden_size, num_experts, inter, top_k, quant, act_dtype, 1, &pl,
                     true);
  if (st != kOk) return st;
  // The router launch does not quantise the hidden rows: the experts read
  // (and, where needed, quantise) them as mstar_fused_moe does.
  pl.route_quant = false;
  pl.one_launch = false;  // nothing clears the sync words before the experts
  if ((st = check_layer_args(pl, activation, workspace, workspace_bytes)) != kOk) return st;
  if (num_tokens == 0) return kOk;
  if (!hidden || !gate_weight || !w1 || !w2 || !out ||
      (quant != MSTAR_QUANT_NONE && (!w1_scale || !w2_scale))) {
    set_last_error("moe_block: null tensor pointer");
    return kInvalidArgument;
  }
  uint8_t* ws = (uint8_t*)workspace;
  float* tw = topk_weights_out ? topk_weights_out : (float*)(ws + pl.off_tw);
  int32_t* ids32 = (int32_t*)(ws + pl.off_ids);
  st = launch_router(hidden, num_tokens, hidden_size, gate_weight, num_experts, top_k, renormalize,
                     tw, ids32, topk_ids_out, logits_out, stream);
  if (st != kOk) return st;
  if (!pl.ids_mode) {
    st = launch_align(ids32, kI32, pl.slots, num_experts, pl.bm, (int32_t*)(ws + pl.off_sorted),
                      (int32_t*)(ws + pl.off_eids), (int32_t*)(ws + pl.off_ntpp), pl.max_padded,
                      (int32_t*)(ws + pl.off_eoff), (int32_t*)(ws + pl.off_ecnt),
                      ws + pl.off_scratch, pl.scratch_bytes, stream);
    if (st != kOk) return st;
  }
  return run_experts(pl, hidden, act_dtype, num_tokens, hidden_size, w1, w2, num_experts, inter,
                     quant, w1_scale, w2_scale, tw, kF32, ids32, kI32, top_k, activation, 1, out,
                     ws, stream);
}

int mstar_moe_route(const void* router_logits, int logits_dtype, int64_t num_tokens,
                    int num_experts, int top_k, int renormalize, float* topk_weights,
                    int32_t* topk_ids_i32, int64_t* topk_ids_i64, int block_size,
                    int32_t* sorted_token_ids, int64_t sorted_len, int32_t* expert_ids,
                    int64_t expert_ids_len, int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                    int32_t* expert_counts, void* scratch, size_t scratch_bytes, void* stream) {
  if (block_size > 0 && expert_ids_len < (sorted_len + block_size - 1) / block_size) {
    set_last_error("moe_route: experts_ids too small");
    return kInvalidArgument;
  }
  return launch_route(router_logits, logits_dtype, num_tokens, num_experts, top_k, renormalize,
                      topk_weights, topk_ids_i32, topk_ids_i64, block_size, sorted_token_ids,
                      expert_ids, num_tokens_post_pad, sorted_len, expert_offsets, expert_counts,
                      scratch, scratch_bytes, (hipStream_t)stream);
}

int mstar_moe_route_scratch_size(int64_t num_tokens, int num_experts, int top_k, size_t* bytes) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0) {
    set_last_error("moe_route_scratch_size: invalid sizes");
    return kInvalidArgument;
  }
  if (bytes) *bytes = route_scratch_bytes(num_tokens, top_k, num_experts);
  return kOk;
}

int mstar_moe_align_scratch_size(int64_t numel, int num_experts, size_t* bytes) {
  if (numel < 0 || num_experts <= 0) {
    set_last_error("moe_align_scratch_size: invalid sizes");
    return kInvalidArgument;
  }
  if (bytes) *bytes = align_scratch_bytes(numel, num_experts);
  return kOk;
}

}  // extern "C"
