// Launch interfaces of the Allie gfx950 kernels (host side of each .hip file).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace allie {

// ---------------------------------------------------------------- timing
// The benchmark's per-kernel timing: while a probe is armed, the next
// probe-aware launch (launch_timed) records the armed events at its own
// start and end on the GPU (hipExtLaunchKernelGGL) and disarms it; other
// launches are untouched.
struct LaunchProbe {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchProbe* launch_probe_take();  // the armed probe (now disarmed), or null
template <typename K, typename... Args>
inline void launch_timed(K kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t st, Args... args) {
  if (LaunchProbe* p = launch_probe_take())
    hipExtLaunchKernelGGL(kernel, grid, block, lds, st, p->start, p->stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

// ---------------------------------------------------------------- packing
struct PackArgs {
  const uint32_t* words;  // flat tokenizer words, games back to back
  const int32_t* lens;    // [B] words per game (before truncation)
  int B, max_len, block, first_block, max_blocks, q_tile;
  int capacity;           // length of ids/pos/seq_of/slot
  int32_t* cu_seqlens;    // [B+1]
  int64_t* in_off;        // [B] word offset of each game (scratch)
  int32_t* ids;           // [T]
  int32_t* pos;           // [T]
  int32_t* seq_of;        // [T]
  int32_t* last_idx;      // [B]
  int32_t* blk_off;       // [B+1]
  int32_t* block_table;   // [B][max_blocks] or null
  int32_t* slot;          // [T] or null
  const int32_t* block_table_in;  // optional [B][max_blocks_in]: slots come from these blocks
  int max_blocks_in;
  int32_t* tiles;         // attention query tiles or null
  int pad_id;             // token id flagged when it occurs inside a game (-1: none)
  int32_t* status;        // [1]: bit 1 empty game, 2 capacity exceeded, 4 table too small,
                          //      8 PAD id inside a game
};
hipError_t launch_pack(const PackArgs& a, hipStream_t st);

// ------------------------------------------------- embedding / LayerNorm
// act_bf16: activations written as bf16 (else fp32); emulate_bf16: apply the
// bf16-autocast rounding points of the reference (Elo control matmul).
struct EmbedArgs {
  const int32_t* ids;
  const int32_t* pos;
  int T, d, vocab;
  int n_positions;    // rows of wpe; positions are clamped into [0, n_positions)
  const float* wte;   // [vocab][d]
  const float* wpe;   // [n_pos][d]
  const float* ctrl;  // [2][d]
  const float* ln_g;  // first block's ln_1
  const float* ln_b;
  float eps;
  float* h;           // [T][d] residual stream (fp32)
  void* x;            // [T][d] LayerNorm output (bf16 or fp32)
  int act_bf16;
};
hipError_t launch_embed_ln(const EmbedArgs& a, hipStream_t st);

struct LNArgs {
  const float* h;          // [rows][d] fp32
  const int32_t* row_idx;  // optional gather: output row r reads h[row_idx[r]]
  int rows, rows_out, d;   // rows_out >= rows: extra rows are zero-filled
  const float* g;
  const float* b;
  float eps;
  void* y;                 // [rows_out][d] bf16 or fp32
  int act_bf16;
  // optional residual add before the norm: row src is h[src] + add[src]
  // (add bf16 [rows][d], bf16 activations only; may alias y, each row is
  // read whole before it is written), written back to h_out[src] when
  // h_out is set (may alias h)
  const void* add;
  float* h_out;
  // optional second addend (bf16 [rows][d], with add set): the row is
  // (h + add) + add2, summed in that order
  const void* add2;
};
hipError_t launch_layernorm(const LNArgs& a, hipStream_t st);

// ------------------------------------------------------------------ GEMM
// C[m, n] = sum_k A[m, k] * W[n, k]   (both operands K-contiguous)
enum Epilogue {
  EPI_STORE = 0,   // y = acc + bias                        -> C
  EPI_GELU = 1,    // y = gelu(acc + bias)                  -> C
  EPI_RESID = 2,   // R[m, n] += acc + bias                 (R fp32, in place)
};
enum WType { W_BF16 = 0, W_F32 = 1, W_FP8 = 2 };

struct GemmArgs {
  const void* A;       // [M][lda] bf16 (W_BF16 / W_FP8) or fp32 (W_F32)
  const void* W;       // [N][K]
  const float* bias;   // [N] or null
  const float* scale;  // [N] per-output-channel weight scale (W_FP8) or null
  void* C;             // [M][ldc] bf16 or fp32
  float* R;            // [M][ldr] residual (EPI_RESID)
  int M, N, K, lda, ldc, ldr;
  int epi;
  int wtype;
  int out_f32;         // store C as fp32 (else bf16)
  int split;           // K splits (MFMA kernels; <= 1: none)
  float* part;         // [split][M][N] fp32 partial sums when split > 1
  void* wdq;           // W_FP8: [N][K] bf16 buffer the weights are widened into for the
                       // persistent kernel (large M), or null
  // An extend's QKV projection (EPI_STORE, N = 3 d): with kv_pool set the key
  // and value columns [d, 3 d) of row m go to pool slot kv_slot[m] of layer
  // kv_layer ([layer][kv_pool_blocks][k|v][head][16][64] bf16) instead of C
  // (the skinny kernel writes them to C as well); rows with a slot outside
  // the pool are not written (see gemm_stores_kv)
  void* kv_pool;
  const int32_t* kv_slot;
  int kv_layer, kv_pool_blocks;
  // Skinny kernel only: with ln_h set, A is not read; the A operand is the
  // LayerNorm of rows of ln_h (fp32 [*][K]; row m is ln_h row ln_row[m], or m
  // when ln_row is null) with gamma ln_g, beta ln_b and eps ln_eps, rounded to
  // bf16.  Every workgroup computes it into LDS with launch_layernorm's lane
  // layout and summation order, so the operand equals what that kernel
  // writes, bit for bit (see gemm_skinny_ln_ok).
  const float* ln_h;
  const int32_t* ln_row;
  const float* ln_g;
  const float* ln_b;
  float ln_eps;
};
hipError_t launch_gemm(const GemmArgs& a, hipStream_t st);
bool gemm_mfma_supported(const GemmArgs& a);
// M <= SKINNY_MAX_M rows, bf16 or fp8 weights: one wave per 4 output columns
// streams the weights once (launch_gemm picks it for such shapes)
constexpr int SKINNY_MAX_M = 8;
bool gemm_skinny_supported(const GemmArgs& a);
// whether an M x N x K GEMM with bf16 or fp8 weights (wtype) runs on the
// skinny kernel with its A operand's LayerNorm in the prologue (ln_h): K a
// multiple of 256 of at most SKINNY_LN_MAX_K
constexpr int SKINNY_LN_MAX_K = 2048;
bool gemm_skinny_ln_ok(int M, int N, int K, int wtype);
hipError_t launch_gemm_skinny(const GemmArgs& a, hipStream_t st);
// true when this GEMM runs on the persistent 256 x 256 kernel (large M,
// bf16 weights or fp8 with wdq, store or gelu epilogue); the forward then writes attention
// and MLP projections with a store epilogue and adds them to the residual
// stream in the following LayerNorm
bool gemm_uses_persistent(const GemmArgs& a);
// true when launch_gemm writes this QKV GEMM's keys and values to a.kv_pool
// itself (MFMA kernels with bf16 output, and the skinny kernel); otherwise the
// caller copies them
bool gemm_stores_kv(const GemmArgs& a);
// block rows of the 256x128-class kernel for an M x N output: 256, 192 or
// 128 (see gemm_tile_m)
int gemm_tile_m(int M, int N);
// K splits the forward uses for an M x N x K MFMA GEMM: enough blocks for
// every CU when the output tiles alone leave most idle (small M)
int gemm_split_factor(int M, int N, int K);

// ------------------------------------------------------------- attention
// Varlen causal self-attention over packed sequences (no KV cache):
// qkv [T][3d] (q | k | v column blocks, heads as head_dim column groups),
// out [T][d].
struct AttnVarlenArgs {
  const void* qkv;
  const int32_t* cu_seqlens;
  const int32_t* tiles;  // (seq << 5) | q_tile, heaviest first (unused by the bf16 path)
  int n_tiles, B, T, n_head, head_dim;
  float scale;
  void* out;
  int act_bf16;
  int32_t* order;        // bf16 path: [B] workspace, games by decreasing length
  int order_ready;       // order already holds this batch's order (later layers)
  int last_only;         // bf16 path: only each game's last row of out is needed (the
                         // other rows may be left unwritten)
};
constexpr int ATTN_Q_TILE = 64;
hipError_t launch_attn_varlen(const AttnVarlenArgs& a, hipStream_t st);

// Paged attention: queries are new tokens of B sequences; keys/values come
// from a paged pool (block = 16 tokens) that already holds the new tokens.
// Pool layout: [layer][pool_blocks][k|v][head][16][head_dim]; slot = block*16 + offset.
constexpr int KV_BLOCK = 16;
struct KVWriteArgs {
  const void* qkv;       // [T][3d]
  const int32_t* slot;   // [T] pool slot (block * 16 + offset); invalid slots are skipped
  int T, n_layer, layer, n_head, head_dim;
  int pool_blocks;       // blocks in the pool (bounds of every slot)
  void* pool;
  int act_bf16;
};
hipError_t launch_kv_write(const KVWriteArgs& a, hipStream_t st);

// Extend attention: n new tokens, in groups (tokens of group g are
// [group_start[g], group_start[g+1])).  Token i of group g attends
//   1. the group's shared prefix: positions 0 .. prefix_len[g]-1, held in the
//      pool blocks prefix_blocks[g][0 ..], and then
//   2. its private keys: the n_extra[i] pool slots extra_slot[i][0 ..] (a
//      search node's ancestors, then the token itself).
// Every key is visible (the causal order is in how the caller builds the
// lists).  Pool layout: [layer][pool_blocks][k|v][head][16][head_dim].  Block ids
// and slots outside the pool are skipped (and flagged by extend_prepare).
struct ExtendAttnArgs {
  const void* qkv;             // [n][3d] new tokens (q | k | v)
  const int32_t* pos;          // [n] token positions: prefix keys at or past pos[i] are not visible
  int n, n_head;
  int one_token_groups;        // wave kernel: token i is group i (all groups of one token)
  const int32_t* group_start;  // [G + 1]
  int n_groups;
  const int32_t* prefix_len;   // [G]
  const int32_t* prefix_blocks;  // [G][max_blocks]
  int max_blocks;
  const int32_t* extra_slot;   // [n][max_extra]
  const int32_t* n_extra;      // [n]
  int max_extra;
  const int32_t* tiles;        // tree kernel: (group << 8) | q_tile of tile_q queries
  int n_tiles, tile_q;         // tile_q: 64 or 128
  const void* pool;            // pool base (the kernel adds the layer offset)
  int pool_blocks, n_layer, layer;
  float scale;
  void* out;                   // [n][d]
  int act_bf16;
  const int32_t* order;        // wave kernel: token of the i-th (token, head) row, or null (identity)
  const int32_t* self_slot;    // tree kernel: [n] each token's own pool slot (its last extra; -1: none)
  int head_group;              // tree kernel: heads per workgroup (set by its launcher)
};
// one wave per (token, head), any group sizes, bf16 or fp32
hipError_t launch_attn_extend_wave(const ExtendAttnArgs& a, hipStream_t st);
// one workgroup of waves per (token, head) of one-token groups (bf16), the
// waves splitting the keys: for batches of at most DECODE_SPLIT_MAX_ROWS
// (token, head) rows, too few to fill the device with one wave per row
constexpr int DECODE_SPLIT_MAX_ROWS = 256;
hipError_t launch_attn_extend_split(const ExtendAttnArgs& a, hipStream_t st);
// order[0 .. n) of the one-token groups 0 .. n - 1, most keys first
hipError_t launch_decode_order(const ExtendAttnArgs& a, int n, int32_t* order, hipStream_t st);
// MFMA tiles of tile_q queries sharing a group's prefix, private keys as
// columns (bf16); needs tiles and self_slot, and a block table of at most
// TREE_MAX_BLOCKS blocks (staged in LDS)
constexpr int TREE_MAX_BLOCKS = 256;
hipError_t launch_attn_extend_tree(const ExtendAttnArgs& a, hipStream_t st);
// Groups g0 .. of at most FAN_MAX_Q tokens each (bf16): one workgroup of
// fan_waves(max_blocks) waves per (group, head), the waves splitting the
// prefix's 64-key chunks
constexpr int FAN_MAX_Q = 16;
constexpr int FAN_MAX_BLOCKS = 512;  // block-table width: 16 chunks of 4 blocks per wave at 8 waves
inline int fan_waves(int max_blocks) {
  const int ch = (max_blocks * KV_BLOCK + 63) / 64;
  return ch < 1 ? 1 : (ch > 8 ? 8 : ch);
}
// groups [g0, g1); waves: 1..8, or 0 for fan_waves(max_blocks)
hipError_t launch_attn_extend_fan(const ExtendAttnArgs& a, int g0, int g1, int waves, hipStream_t st);
// tiles[] = (g << 8) | t for every tile_q-query tile t of every group g in
// [first_group, n_groups), in order
hipError_t launch_extend_tiles(const int32_t* group_start, int first_group, int n_groups, int tile_q, int32_t* tiles,
                               hipStream_t st);

// Validates an extend batch and derives each token's own pool slot (the last
// of its extras).  status bits: 1 n_extra outside [1, max_extra], 2 a block id
// or slot outside the pool, 4 a position outside [0, n_positions).
struct ExtendPrepArgs {
  int n, n_groups, max_blocks, max_extra, pool_blocks, n_positions;
  const int32_t* pos;
  const int32_t* group_start;
  const int32_t* prefix_len;
  const int32_t* prefix_blocks;
  const int32_t* extra_slot;
  const int32_t* n_extra;
  int32_t* self_slot;          // [n]
  int32_t* status;             // [1], written (not accumulated)
};
hipError_t launch_extend_prepare(const ExtendPrepArgs& a, hipStream_t st);

// ----------------------------------------------------------------- heads
// logits/value/time from the heads GEMM output rows, plus softmax summary.
struct HeadsArgs {
  const float* z;        // [B][ldz] fp32 heads GEMM output (acc + bias)
  int B, ldz, vocab, n_moves;
  int value_col, time_col;
  float temperature;     // the reference clamps it to >= 1e-5 (decode.py:191)
  const uint32_t* legal; // optional [B][legal_words] bitmask over move ids
  int legal_words;
  float* logits;         // [B][vocab] or null
  float* logits_raw;     // [B][vocab] z before the bf16 rounding, or null
  float* value;          // [B]
  float* time;           // [B]
  int32_t* top1;         // [B]
  float* lse;            // [B] logsumexp of logits[:n_moves] * inv_temp (masked)
  float* max_logit;      // [B]
  int emulate_bf16;
};
hipError_t launch_heads(const HeadsArgs& a, hipStream_t st);

// -------------------------------------------------------- weight packing
// dst[n][k] = src[k][n] (Conv1D [in,out] -> [out,in]); bf16 or fp32 dst.
hipError_t launch_transpose_convert(const float* src, int rows, int cols, void* dst, int dst_bf16,
                                    int ld_dst, hipStream_t st);
hipError_t launch_convert(const float* src, int64_t n, void* dst, int dst_bf16, int round_bf16,
                          hipStream_t st);

// dst row r = src row idx[r] (rows of row_bytes, a multiple of 16)
hipError_t launch_gather_rows(const void* src, const int32_t* idx, int rows, int row_bytes, void* dst,
                              hipStream_t st);

}  // namespace allie
