// Host-side launchers shared between the kernel translation units and the
// C-ABI layer.  Every launcher validates its arguments, enqueues on the
// stream it is given and returns a Status code; nothing allocates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mstar {

// launch_state.hip: per-device launch state, safe from several host threads.
// CU count of the current device (cached per device); 0 with the error
// message set if the device cannot be read (hipGetDevice failing).
int device_cu_count();
// Opt `kernel` into `bytes` of dynamic LDS on the current device (once per
// device and size); kOk or kLaunchError with the message set.
int ensure_dynamic_lds(const void* kernel, size_t bytes, const char* what);
// Resident workgroups per CU of `kernel` at this block size and LDS size on
// the current device (cached per device, kernel, block size and LDS size);
// 0 with the error message set if the device cannot be read.
int occupancy_per_cu(const void* kernel, int threads, size_t lds_bytes);

// route.hip
// With `hidden` (bf16 [M, H], H % 512 == 0) the launch also quantises the
// hidden rows per group of 128: hq [M, H] holds the e4m3fn values widened to
// bf16, hs [M, H/128] the scales.
// Fused router (router.hip): bf16 hidden [M, H] x bf16 gate weight [E, H]
// -> bf16 logits (optionally stored), softmax top-k, renormalisation.
int launch_router(const void* hidden, int64_t M, int64_t H, const void* gate_weight, int E, int k,
                  int renorm, float* w, int32_t* ids32, int64_t* ids64, void* logits_out,
                  hipStream_t stream);
// zero / n_zero: words the launch clears (for the launch after it).
int launch_topk_softmax(const void* logits, int logits_dtype, int64_t M, int E, int k,
                        int renorm, float* w, int32_t* ids32, int64_t* ids64, hipStream_t stream,
                        const void* hidden = nullptr, int64_t H = 0, uint16_t* hq = nullptr,
                        float* hs = nullptr, int* zero = nullptr, int n_zero = 0);
// Alignment: one workgroup for numel <= 4096 (or without scratch), otherwise
// a histogram pass and a scan+scatter pass over align_scratch_bytes() of
// scratch.  Deterministic (slots ascend within an expert) either way.
int launch_align(const void* ids, int ids_dtype, int64_t numel, int E, int bm,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, int64_t max_padded,
                 int32_t* expert_off, int32_t* expert_cnt, void* scratch, size_t scratch_bytes,
                 hipStream_t stream);
size_t align_scratch_bytes(int64_t numel, int E);
// Softmax top-k + alignment: one launch for M*k <= 4096, else two
// (top-k + per-workgroup histograms, then scan + scatter); the latter needs
// route_scratch_bytes() of scratch.
int launch_route(const void* logits, int logits_dtype, int64_t M, int E, int k, int renorm,
                 float* w, int32_t* ids32, int64_t* ids64, int bm, int32_t* sorted_ids,
                 int32_t* expert_ids, int32_t* ntpp, int64_t max_padded, int32_t* expert_off,
                 int32_t* expert_cnt, void* scratch, size_t scratch_bytes, hipStream_t stream,
                 const void* hidden = nullptr, int64_t H = 0, uint8_t* hq = nullptr,
                 float* hs = nullptr);
size_t route_scratch_bytes(int64_t M, int k, int E);
// Whether launch_route takes the multi-workgroup path for M tokens (the one
// that can quantise the hidden rows on the way).
bool route_is_grid(int64_t M, int k);

// quant.hip
// widen: q receives the e4m3fn values widened to bf16 (2 bytes per element).
int launch_quant_fp8_group(const void* x, int x_dtype, int64_t rows, int64_t cols,
                           int64_t ld_x, void* q, float* s, hipStream_t stream, bool widen = false);
int launch_quant_fp8_row(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q,
                         float* s, hipStream_t stream);

// elementwise.hip
int launch_act_and_mul(const void* gate_up, void* out, int dtype, int64_t rows, int64_t inter,
                       int activation, hipStream_t stream);
int launch_sum_reduce(const void* in, void* out, int dtype, int64_t tokens, int64_t topk,
                      int64_t hidden, float scale, hipStream_t stream);
// The same sum over rows stored by sorted position: row j of token t is
// in[pos_of[t * topk + j]].
int launch_sum_reduce_pos(const void* in, const int32_t* pos_of, void* out, int dtype,
                          int64_t tokens, int64_t topk, int64_t hidden, hipStream_t stream);

// moe_gemm.hip --------------------------------------------------------------
// Operand encodings.
enum AKind : int { A_H16 = 0, A_FP8G = 1, A_FP8R = 2 };
enum BKind : int { B_H16 = 0, B_FP8BLK = 1, B_INT4G = 2, B_FP8R = 3 };
enum EpiKind : int { EPI_STORE = 0, EPI_ACT = 1, EPI_DENSE = 2 };

struct GemmArgs {
  // A: activations, rows of K elements (bytes for fp8), row stride lda.
  const void* A;
  int64_t lda;
  const float* a_scale;  // A_FP8G: [rows, K/128] (stride ld_as); A_FP8R: [rows]
  int64_t ld_as;
  // B: weights [E][N][K] (B_INT4G: [E][N][K/8] int32 words).
  const void* B;
  int64_t ldb;        // row stride in elements (int4: int32 words)
  int64_t b_estride;  // expert stride in elements (int4: words)
  const void* b_scale;  // B_FP8BLK: fp32 [E][ceil(N/128)][K/128]; B_INT4G: 16-bit [E][N][K/128];
                        // B_FP8R: fp32 [N]
  int64_t bs_estride;
  int64_t bs_ld;
  void* C;
  int64_t ldc;
  const void* topk_w;  // per slot routing weight (EPI_STORE with mul_routed)
  int topk_w_dtype;
  const int32_t* sorted_ids;  // grouped mode
  const int32_t* expert_ids;
  const int32_t* ntpp;
  const int32_t* expert_off;  // streaming mode: [E+1] padded starts
  const int32_t* expert_cnt;  // streaming mode: [E] real counts
  int64_t M;          // dense: rows; grouped: number of valid slots (numel)
  int N, K;
  int top_k;          // A row = slot / top_k
  int inter;          // EPI_ACT: gate/up split (N == 2 * inter)
  int mul_routed;
  int activation;     // 0 silu, 1 gelu
  int num_experts;
  int m_blocks;       // grouped: number of m-blocks (expert_ids length)
  // EPI_ACT of the 256-row FP8 kernel: when set, the activation output is
  // quantised per token and group of 128 columns in the epilogue (e4m3fn
  // codes cq [rows, inter], fp32 scales cs [rows, inter/128]) instead of
  // being stored to C.
  uint8_t* cq;
  float* cs;
  // Streaming FP8 kernels only: when set, the per-expert slot lists are
  // built from these [M] router ids (int32 or int64, ids_dtype) instead of
  // sorted_ids / expert_off / expert_cnt.
  const void* topk_ids;
  int ids_dtype;
  // A_FP8G rows hold the e4m3fn values widened to bf16 (2 bytes per
  // element, lda in elements) instead of e4m3fn bytes.
  int a_q16;
  // Grouped 256-row FP8 kernel only: intermediates indexed by sorted
  // position (m-block * 256 + row of the block in sorted_ids) instead of by
  // slot, so that a tile's rows are contiguous.  pos_out: C / cq / cs rows
  // are positions (padding rows are not written); pos_in: A and a_scale rows
  // are positions.  pos_of: when set, the tiles of n-tile 0 record
  // pos_of[slot] = position.
  int pos_out, pos_in;
  int32_t* pos_of;
};

// Tiled grouped / dense GEMM (LDS-staged MFMA tiles); bm is the row block.
int launch_tile_gemm(const GemmArgs& a, int akind, int bkind, int epi, int dtype, bool grouped,
                     int bm, hipStream_t stream);
// Weight-streaming grouped GEMM for small token counts (one workgroup per
// (expert, n-tile); each weight byte is read once).  A_H16 with B_FP8BLK
// quantises the activations per 128-group on the fly.
int launch_stream_gemm(const GemmArgs& a, int akind, int bkind, int epi, int dtype,
                       int max_rows, hipStream_t stream);
bool stream_gemm_supported(int K, int max_rows, int akind, int bkind);

// W4A16 decode (router-ids mode): the CU-resident streaming kernel over
// int4 weights (group-128 bf16 scales) and bf16 token rows.
int launch_stream_int4_cu(const GemmArgs& a, int epi, hipStream_t stream);
// gemm_fp8.hip: persistent FP8 GEMM over tiles of bm (256 or 128) token rows
// x 256 weight rows (8 waves, double-buffered LDS); grouped, bm is the
// alignment block size.
int launch_gemm_fp8_big(const GemmArgs& a, int epi, bool grouped, int bm, hipStream_t stream);
// gemm_w4.hip: W4A16 grouped GEMM over alignment blocks of 64 tokens.  Token
// rows (A) are stored in the int4 codes' pair order (each 8-group holds
// elements 0, 4, 1, 5, 2, 6, 3, 7) with fp32 sums per 128-group (xs,
// [rows, K / 128]).  EPI_ACT writes C in that order and the sums of its
// groups (xs_out, [slots, inter / 128]) for the down GEMM.
// gemm_dense.hip: per-token x per-channel FP8 GEMM for M <= 32 (weights
// streamed once; persistent, one workgroup per CU).
bool dense_stream_supported(int64_t M, int64_t N, int64_t K);
int launch_dense_stream(const GemmArgs& a, hipStream_t stream);
bool w4_tile_supported(int64_t H, int64_t I);
int launch_w4_tile(const GemmArgs& a, int epi, const float* xs, float* xs_out, hipStream_t stream);
// Hidden rows [rows, H] (row stride ldx) -> pair order [rows, H] and the
// group sums [rows, H / 128].
int launch_w4_prep(const void* x, int64_t ldx, int64_t rows, int64_t H, void* out, float* xs,
                   hipStream_t stream);
constexpr int kBigBlockM = 256;

// stream_fp8.hip: persistent FP8 weight streaming (bf16 activations,
// quantised per 128-group on the fly).  exact: reduce each 128-block with
// bf16 MFMAs on the exactly widened FP8 values (fp32-exact accumulation);
// otherwise with the FP8 MFMA.
int launch_stream_fp8(const GemmArgs& a, int epi, bool exact, hipStream_t stream);
constexpr int64_t kStreamMaxIdsSlots = 1024;  // slots a launch in ids mode can take
// The decode layer's gate_up and down streaming GEMMs in one launch (g1:
// gate_up on the routing launch's widened FP8 token rows, or int4 on bf16
// hidden rows; g2: down on g1's bf16 output).  sync_words: at least
// layer_sync_words(E, CU count) ints, zero when the launch starts (the
// routing launch clears them).
bool stream_layer_supported(int64_t H, int64_t I, int64_t slots, int E, bool int4);
int launch_stream_layer(const GemmArgs& g1, const GemmArgs& g2, bool int4, int* sync_words, hipStream_t stream);
// Sync words a layer launch of `nwg` workgroups reads (per-expert counters,
// the error word, per-range claim words).
int layer_sync_words(int E, int nwg);
constexpr int kLayerSyncMaxCus = 1024;
// Test hook: the mode of the layer launches enqueued from now on.
int set_layer_test_mode(int mode);
// mstar_moe_layer with the one-launch decode layer allowed or not.
int moe_layer_impl(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                   const void* router_logits, int logits_dtype, int renormalize, const void* w1,
                   const void* w2, int num_experts, int64_t inter, int quant,
                   const void* w1_scale, const void* w2_scale, int top_k, int activation,
                   void* out, float* topk_weights_out, int64_t* topk_ids_out, void* workspace,
                   size_t workspace_bytes, void* stream, bool allow_one_launch);
// Waits of the layer kernel that gave up on the current device (synchronous copy).
int layer_wait_failures(int* count);
bool stream_fp8_supported(int K, int N, int inter, int epi);


}  // namespace mstar
