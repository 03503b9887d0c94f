/*
 * allie_amd -- C ABI of the MI355X (gfx950) engine for Allie's batched
 * policy/value inference path.
 *
 * The reference (y0mingzhang/allie) is pure Python and has no FFI; its
 * boundary is the model call `model(**batch) -> dict` of
 * CausalLMWithRegressionHead.forward (src/modeling/model.py:85-147), fed by
 * UCITokenizer.pad_and_collate (src/modeling/data.py:281-337) and read by the
 * decode strategies at src/evaluation/decode.py:199-238,356-373.  Each entry
 * point below names the part of that boundary it replaces.  The Python host
 * side (allie_amd/capi.py) binds these symbols with ctypes.
 *
 * Conventions
 *   - every pointer argument is device memory unless its name ends in _host;
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 *   - calls are stream-ordered, never synchronise the device and never
 *     allocate device memory: the caller passes workspaces (sizes from the
 *     *_workspace_bytes queries).  Only allie_model_create allocates (the
 *     weight arena, freed by allie_model_destroy);
 *   - return 0 on success or a negative ALLIE_ERR_* code; the message of the
 *     last failure on the calling thread is allie_last_error().
 */
#ifndef ALLIE_AMD_H
#define ALLIE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ALLIE_OK = 0,
  ALLIE_ERR_ARG = -1,        /* bad argument or shape */
  ALLIE_ERR_HIP = -2,        /* a HIP runtime call failed */
  ALLIE_ERR_NOMEM = -3,      /* weight arena allocation failed */
  ALLIE_ERR_STATE = -4,      /* model not finalised / weight missing */
  ALLIE_ERR_WORKSPACE = -5,  /* workspace too small */
  ALLIE_ERR_LENGTH = -6      /* a game is empty or a table is too small */
};

/* Token id of <PAD> (src/modeling/data.py:197-198: moves, 24 time
 * controls, the resign token, then <BOS> <EOS> <UNK> <PAD>). */
#define ALLIE_PAD_ID 1996

/* Numeric modes. */
enum {
  ALLIE_MODE_FP32 = 0, /* fp32 weights and activations (fp32 check mode) */
  ALLIE_MODE_BF16 = 1, /* bf16 GEMM operands, fp32 residual (torch autocast bf16) */
  ALLIE_MODE_FP8W = 2  /* fp8 e4m3 per-output-channel weights, bf16 activations */
};

typedef struct allie_config {
  int32_t n_layer, d_model, n_head, vocab_size, n_positions, max_length;
  float eps;
  int32_t mode;
} allie_config;

typedef struct allie_model allie_model;

/* Weight kinds, in the reference's state-dict terms (see weights.py). */
enum {
  ALLIE_W_WTE = 0,   /* model.model.transformer.wte.weight [vocab][d]   */
  ALLIE_W_WPE,       /* model.model.transformer.wpe.weight [n_pos][d]   */
  ALLIE_W_CTRL,      /* model.control_embeds.weight [2][d]              */
  ALLIE_W_LNF_G,     /* model.model.transformer.ln_f.weight [d]         */
  ALLIE_W_LNF_B,
  ALLIE_W_VALUE_W,   /* value_head.0.weight [1][d]                      */
  ALLIE_W_VALUE_B,   /* value_head.0.bias [1]                           */
  ALLIE_W_TIME_W,    /* time_head.0.weight [1][d]                       */
  ALLIE_W_TIME_B,
  ALLIE_W_LN1_G = 16,/* per layer: ...h.{i}.ln_1.weight [d]             */
  ALLIE_W_LN1_B,
  ALLIE_W_QKV_W,     /* ...attn.c_attn.weight [d][3d] (Conv1D in x out) */
  ALLIE_W_QKV_B,
  ALLIE_W_O_W,       /* ...attn.c_proj.weight [d][d]                    */
  ALLIE_W_O_B,
  ALLIE_W_LN2_G,
  ALLIE_W_LN2_B,
  ALLIE_W_FC_W,      /* ...mlp.c_fc.weight [d][4d]                      */
  ALLIE_W_FC_B,
  ALLIE_W_PR_W,      /* ...mlp.c_proj.weight [4d][d]                    */
  ALLIE_W_PR_B
};

const char* allie_last_error(void);
int allie_abi_version(void);

/* Model lifetime.  Replaces initialize_model + load_state_dict
 * (src/modeling/model.py:155-198, src/evaluation/evaluate.py:236-243). */
int allie_model_create(const allie_config* cfg, allie_model** out);
void allie_model_destroy(allie_model* m);
/* src: fp32 tensor in the reference's layout (Conv1D weights [in][out]),
 * rows x cols; converted and repacked into the model's arena. */
int allie_model_set_weight(allie_model* m, int kind, int layer, const float* src, int64_t rows,
                           int64_t cols, void* stream);
/* fp8 mode only, for the four block GEMM weights: q [out][in] e4m3fn bytes,
 * scale [out] fp32 (w[in][out] ~= q[out][in] * scale[out]). */
int allie_model_set_weight_fp8(allie_model* m, int kind, int layer, const uint8_t* q,
                               const float* scale, int64_t out_features, int64_t in_features,
                               void* stream);
/* Checks that every weight was set; required before any forward call. */
int allie_model_finalize(allie_model* m);
/* Thresholds of the two-stream split (bf16 modes): a prefill or an extend of
 * at least `tokens` tokens, or an extend with at least `decode_tokens`
 * one-token groups (decode steps), runs as two halves on two streams of the
 * model's own (see allie_prefill and allie_extend); 0 turns that split off.
 * Defaults 24,576 and 512.  No reference counterpart: a tuning knob for
 * callers that run their own streams.  Workspace sizes reported afterwards
 * follow the new thresholds. */
int allie_model_set_split_tokens(allie_model* m, int64_t tokens, int64_t decode_tokens);
/* Heads per workgroup of the tree attention kernel (bf16 extends whose groups
 * exceed 16 tokens, with at most 8 private keys per token): 0 (the default)
 * picks, for 128-query tiles (some group over 64 tokens), the largest of 16,
 * 8, 4, 2 dividing the head count that still leaves at least 1,024
 * workgroups, else one head; a divisor of the head count up to 16 forces it.
 * Every head's arithmetic is the same whatever the grouping, so the results
 * are the same bits.  No reference counterpart: a tuning knob. */
int allie_model_set_tree_heads(allie_model* m, int heads);

/* Ragged packing (replaces the padding half of pad_and_collate,
 * src/modeling/data.py:281-337, for a flat word stream).
 * words: games back to back; lens[n_seq]: words per game before the
 * truncation to max_len (data.py:290).  Outputs are sized by the caller:
 * cu_seqlens[n_seq+1], last_idx[n_seq], blk_off[n_seq+1],
 * block_table[n_seq][max_blocks] (may be NULL), and ids/pos/seq_of/slot
 * [capacity] (slot may be NULL).  in_off is int64 scratch [n_seq].
 * status[1] is written 0 on success, else a bitmask: 1 empty game,
 * 2 capacity exceeded (excess tokens dropped), 4 block table too small,
 * 8 the id pad_id occurs inside a game (pass -1 to skip the check; the
 * reference would mask such a token, data.py:321, the packer keeps it). */
int allie_pack_ragged(const uint32_t* words, const int32_t* lens, int n_seq, int max_len,
                      int block, int first_block, int max_blocks, int capacity,
                      int32_t* cu_seqlens, int64_t* in_off, int32_t* ids, int32_t* pos,
                      int32_t* seq_of, int32_t* last_idx, int32_t* blk_off,
                      int32_t* block_table, int32_t* slot, int pad_id, int32_t* status,
                      void* stream);

/* Outputs of a forward, one entry per game (the values the decode
 * strategies read from out["logits"][:, -1], out["value_logits"][:, -1],
 * out["time_logits"][:, -1], decode.py:204-226).  top1 follows the
 * reference's argmax of softmax(logits / T) (decode.py:223-226): a NaN or
 * +inf among the considered logits gives top1 = the first considered move
 * id and max_logit = lse = NaN. */
typedef struct allie_outputs {
  float* logits;     /* [n_seq][vocab] or NULL */
  float* value;      /* [n_seq] tanh value head */
  float* time;       /* [n_seq] time head (normalised units) */
  int32_t* top1;     /* [n_seq] first argmax over (legal) move logits / T */
  float* max_logit;  /* [n_seq] that maximum (of logits / T) */
  float* lse;        /* [n_seq] logsumexp of (legal) move logits / T */
  float* logits_raw; /* [n_seq][vocab] fp32 logits before the final bf16
                        rounding of the bf16 modes, or NULL */
} allie_outputs;

/* Batched prefill forward: replaces `model(**pad_and_collate(games))` plus
 * the last-token reads of Policy.score_full (decode.py:199-226).
 * words: device word stream; lens_host: host array [n_seq].
 * legal: optional [n_seq][legal_words] bitmask over move ids (NULL = all).
 * kv_pool: optional paged KV pool of kv_pool_blocks blocks (layout
 * [layer][kv_pool_blocks][k|v][head][16][head_dim], activation dtype; the
 * layout depends on the block count, so every call on one pool must pass the
 * same kv_pool_blocks, its true size) that receives
 * every layer's keys and values (NULL = no cache).  Game i's position p goes
 * to block kv_block_table[i][p / 16] (device int32 [n_seq][kv_max_blocks],
 * entries -1 or outside the pool are not written) when that table is given,
 * else to the contiguous blocks first_block + blk_off[i] ...
 * status (device int32[1], optional) receives the packer's bitmask (see
 * allie_pack_ragged): 4 a game longer than its kv_block_table row (its tail
 * is not cached), 8 the <PAD> id inside a game (the reference's padded batch
 * would mask that token, data.py:321; here it is an ordinary token).
 * A bf16 prefill of at least 24,576 tokens (allie_model_set_split_tokens)
 * with neither kv_pool nor status
 * runs as two halves of consecutive games on two streams of its own, forked
 * from and joined back into `stream` (results as for one piece: rows never
 * interact across games); it needs the workspace that
 * allie_prefill_workspace_bytes reports, and runs in one piece on less. */
size_t allie_prefill_workspace_bytes(const allie_model* m, int n_seq, int n_tokens);
size_t allie_kv_block_bytes(const allie_model* m);
int allie_prefill(allie_model* m, const uint32_t* words, const int32_t* lens_host, int n_seq,
                  float temperature, const uint32_t* legal, int legal_words,
                  const allie_outputs* out, void* kv_pool, int kv_pool_blocks, int first_block,
                  const int32_t* kv_block_table, int kv_max_blocks, int32_t* status,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Extend: the forward of n_tok NEW tokens over a paged KV cache -- one
 * decode step of many games, or one level of MCTS children.  Replaces the
 * full-prefix recompute that MCTS.evaluate_node runs per leaf
 * (src/evaluation/decode.py:356-373, "no kv caching", README.md:80) and that
 * Policy.score_full runs per appended move (decode.py:199-203): the result at
 * a new token equals that recompute's last-token output.
 *
 * Tokens come in n_groups contiguous groups: group g is tokens
 * [group_start_host[g], group_start_host[g+1]) (HOST array, read during the
 * call).  Token i of group g attends
 *   1. the group's shared prefix, positions 0 .. min(prefix_len[g], pos[i])-1,
 *      stored in the pool blocks prefix_blocks[g][0 .. ceil(prefix_len[g]/16)-1]
 *      (a token placed inside its group's prefix sees only earlier positions),
 *      then
 *   2. its own keys: pool slots extra_slot[i][0 .. n_extra[i]-1] (a search
 *      node's ancestors in root-to-leaf order, then the node itself).
 * Every layer's key/value of token i is written to pool slot
 * extra_slot[i][n_extra[i]-1] (slot = block * 16 + offset) before attention.
 * ids/pos: the token id and its position (0-based, = number of keys before
 * it).  All of ids, pos, prefix_len, prefix_blocks, extra_slot, n_extra are
 * device int32 arrays; outputs are per token as in allie_prefill.
 * status (device int32[1], optional) is written with 1 a token's n_extra
 * outside [1, max_extra], 2 a block id or slot outside the pool, 4 a position
 * outside the model's positions; keys in bad blocks are skipped, never read.
 * Groups may hold at most 16384 tokens; a batch with a group of several
 * tokens after its leading one-token groups takes block tables of at most 512
 * blocks (max_blocks), and of at most 256 blocks (4096 positions) with a
 * group of more than 16 tokens (ALLIE_ERR_ARG otherwise).  A new game's whole prefix of P
 * tokens is one group with prefix_len P over the game's own blocks, token t
 * at pos t with its own slot (position t) as its only extra: every layer
 * writes the P keys before attention, and token t sees positions 0..t.  A
 * batch may mix such groups with decode steps; one-token groups placed first
 * are streamed by the decode kernel, the rest share their group's keys
 * across query tiles.
 * A bf16 extend of at least 24,576 tokens, or with at least 512 leading
 * one-token groups (allie_model_set_split_tokens), runs as two halves of
 * consecutive groups on the model's two streams, forked from and joined back
 * into `stream`, the halves' flags OR-ed into status; it needs the workspace
 * that allie_extend_workspace_bytes reports, and runs in one piece on less. */
size_t allie_extend_workspace_bytes(const allie_model* m, int n_tok, int n_groups);
int allie_extend(allie_model* m, const int32_t* ids, const int32_t* pos, int n_tok,
                 const int32_t* group_start_host, int n_groups, const int32_t* prefix_len,
                 const int32_t* prefix_blocks, int max_blocks, const int32_t* extra_slot,
                 const int32_t* n_extra, int max_extra, float temperature, const uint32_t* legal,
                 int legal_words, const allie_outputs* out, void* kv_pool, int kv_pool_blocks,
                 int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free extend.  No counterpart in the reference: an addition for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight search/serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as allie_extend, except:
 *   - no workspace: the call's scratch (activations, K-split partial sums,
 *     tables) lives in a file-scope device array of
 *     ALLIE_NOALLOC_SCRATCH_BYTES that each GPU holds until the process
 *     ends (its per-device address is looked up in allie_model_create);
 *   - group_start: the DEVICE copy of group_start_host (int32 [n_groups+1]),
 *     so no host-to-device staging is needed; group_start_host is still read
 *     on the host to plan the call;
 *   - at most ALLIE_NOALLOC_MAX_TOKENS tokens, and the call's scratch layout
 *     must fit the array (ALLIE_ERR_WORKSPACE otherwise; every shipped shape
 *     -- small, medium, the 2x fp8 shape -- fits at the maximum).
 * It calls no hipMalloc/hipFree/hipHostMalloc.  All calls on one GPU share
 * that GPU's array, which keeps the last call's contents (nothing in it must
 * start at zero): calls that overlap on one GPU (different streams or host
 * threads without ordering) race and must not be issued. */
#define ALLIE_NOALLOC_SCRATCH_BYTES (32u << 20)
#define ALLIE_NOALLOC_MAX_TOKENS 256
int allie_extend_noalloc(allie_model* m, const int32_t* ids, const int32_t* pos, int n_tok,
                         const int32_t* group_start_host, const int32_t* group_start, int n_groups,
                         const int32_t* prefix_len, const int32_t* prefix_blocks, int max_blocks,
                         const int32_t* extra_slot, const int32_t* n_extra, int max_extra, float temperature,
                         const uint32_t* legal, int legal_words, const allie_outputs* out, void* kv_pool,
                         int kv_pool_blocks, int32_t* status, void* stream);

/* Kernel probe for benchmarks: while active, the main kernel of every op of
 * one kind inside allie_prefill / allie_extend records HIP events at its own
 * start and end on the GPU (hipExtLaunchKernelGGL); allie_probe_end waits for
 * them and returns the summed duration and the count (a GEMM with fp8 weights
 * on the persistent path: from the start of its widening kernel to the end of
 * the product).  Not re-entrant; the
 * probed calls must all be on one device.  No counterpart in the reference. */
enum {
  ALLIE_PROBE_QKV = 0,  /* QKV projection GEMM */
  ALLIE_PROBE_PROJ,     /* attention output projection GEMM */
  ALLIE_PROBE_FC,       /* MLP c_fc GEMM + gelu */
  ALLIE_PROBE_FC2,      /* MLP c_proj GEMM */
  ALLIE_PROBE_ATTN,     /* attention of a layer (prefill: varlen kernel; extend: the fan or tree kernel,
                           else the decode kernel) */
  ALLIE_PROBE_DECODE    /* extend: the one-token-group (decode) attention kernel */
};
int allie_probe_begin(int kind, int max_launches);
/* Before allie_probe_end: the time during which at least one probed launch
 * ran (the union of their [start, end] intervals), which differs from the
 * summed durations when launches on different streams overlap (a prefill
 * split into two halves). */
int allie_probe_span(float* span_ms_host);
int allie_probe_end(float* total_ms_host, int* n_launches_host);

/* Building blocks exported for tests and benchmarks.
 * GEMM: C[m][n] (+)= sum_k A[m][k] W[n][k] with the engine's epilogues
 * (0 store, 1 gelu, 2 residual add into R fp32); wtype 0 bf16, 1 fp32, 2 fp8.
 * wdq: fp8 only, optional device buffer of N * K bf16 that large-M GEMMs
 * widen the weights into for the persistent kernel (the forward's path).
 * Shapes (bf16 / fp8): N % 128 == 0 and K % 32 == 0, or M <= 8 rows with
 * N % 4 == 0 and K % 8 == 0 (the skinny kernel, which such M always use). */
int allie_gemm(const void* A, const void* W, const float* bias, const float* scale, void* C,
               float* R, int M, int N, int K, int epi, int wtype, int out_f32, void* wdq, void* stream);
/* The same GEMM with K split into split_k parts (0: the split the forward
 * picks for this shape, allie_gemm_split_factor) whose fp32 partial sums go
 * to part (split * M * N floats), then one reduction pass applies the
 * epilogue.  bf16 or fp8 weights.  The forward splits small-M GEMMs this way
 * (decode steps, tree levels: the output tiles alone would leave most CUs
 * idle); the split count is fixed per shape, so results are deterministic. */
int allie_gemm_splitk(const void* A, const void* W, const float* bias, const float* scale, void* C,
                      float* R, int M, int N, int K, int epi, int wtype, int out_f32, int split_k,
                      float* part, size_t part_bytes, void* stream);
int allie_gemm_split_factor(int M, int N, int K);
/* Varlen causal attention over packed games (qkv [T][3 H 64] -> out [T][H 64]).
 * bf16: order_ws is device workspace of n_seq int32 (games by length), every
 * game at most 512 tokens; fp32: tiles/order_ws unused. */
int allie_attn_varlen(const void* qkv, const int32_t* cu_seqlens, const int32_t* tiles,
                      int n_tiles, int n_seq, int n_tokens, int n_head, int head_dim,
                      float scale, void* out, int act_bf16, int32_t* order_ws, void* stream);
int allie_layernorm(const float* h, const int32_t* row_idx, int rows, int rows_out, int d,
                    const float* g, const float* b, float eps, void* y, int act_bf16,
                    void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ALLIE_AMD_H */
