// C ABI and host runtime of the engine: model object and weight arena,
// workspace layout, and the prefill orchestration.  Declarations and the
// reference interfaces each entry point replaces are in include/allie_amd.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/allie_amd.h"
#include "kernels.hpp"

using namespace allie;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                                  \
  do {                                                                                 \
    hipError_t _e = (expr);                                                            \
    if (_e != hipSuccess) return fail(ALLIE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

struct LayerW {
  float *ln1_g, *ln1_b, *b_qkv, *b_o, *ln2_g, *ln2_b, *b_fc, *b_pr;
  void *w_qkv, *w_o, *w_fc, *w_pr;
  float *s_qkv, *s_o, *s_fc, *s_pr;  // fp8 scales
};

constexpr int N_KINDS = 32;

// Kernel probe: for every op of one kind inside the forward, the op's main
// kernel launch records a pair of HIP events at its own start and end, for
// the benchmark's roofline figure (process-wide, not re-entrant).
struct Probe {
  int kind = -1;
  int n = 0;
  std::vector<hipEvent_t> start, stop;
  LaunchProbe armed;
  bool is_armed = false, taken = false;
} g_probe;

hipError_t probe_mark(int kind, bool before, hipStream_t st) {
  (void)st;
  if (g_probe.kind != kind) return hipSuccess;
  if (before) {
    if (g_probe.n >= (int)g_probe.start.size()) return hipSuccess;
    g_probe.armed.start = g_probe.start[g_probe.n];
    g_probe.armed.stop = g_probe.stop[g_probe.n];
    g_probe.is_armed = true;
    g_probe.taken = false;
    return hipSuccess;
  }
  if (g_probe.taken) ++g_probe.n;  // an op without a probe-aware launch is not counted
  g_probe.is_armed = g_probe.taken = false;
  return hipSuccess;
}

// Device scratch of allie_extend_noalloc: file-scope device memory, so that
// entry point never allocates.  Every device the library runs on holds its
// own copy until the process ends.  In host code `scratch` is only a handle
// for hipGetSymbolAddress; the device address of each GPU's copy is looked up
// once per device (scratch_init, from allie_model_create with that device
// current) and only that address is passed to kernels.
__device__ __align__(256) char scratch[ALLIE_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// Records the current device's address of `scratch` (idempotent).
hipError_t scratch_init(int dev) {
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return hipSuccess;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  g_scratch_ptr[dev] = p;
  return hipSuccess;
}

void* scratch_ptr(int dev) {
  if (dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return g_scratch_ptr[dev];
}

}  // namespace

namespace allie {
LaunchProbe* launch_probe_take() {
  if (!g_probe.is_armed) return nullptr;
  g_probe.is_armed = false;
  g_probe.taken = true;
  return &g_probe.armed;
}
}  // namespace allie

// Pinned host staging for the small host arrays of a call (lengths, group
// starts): a copy from pageable memory would synchronise the stream, so the
// array is copied into one of a ring of pinned buffers and uploaded from
// there.  An event recorded after each upload guards the buffer's reuse.
struct PinnedRing {
  static constexpr int N = 4;
  int32_t* buf[N] = {};
  size_t cap[N] = {};
  hipEvent_t ev[N] = {};
  bool used[N] = {};
  int next = 0;
};

struct allie_model {
  allie_config cfg;
  int device = 0;          // the device current at allie_model_create (owns the arena)
  PinnedRing pinned;
  int d, H, hd, L, V, NH;  // NH: rows of the heads matrix (vocab + 2, padded)
  int wsz;                 // bytes per block-GEMM weight element
  int hsz;                 // bytes per heads-matrix element
  int act_bf16;
  char* arena = nullptr;
  size_t arena_bytes = 0;
  float *wte, *wpe, *ctrl, *lnf_g, *lnf_b, *b_head;
  void* w_head;
  std::vector<LayerW> layers;
  std::vector<uint8_t> set;  // [(L + 1) * N_KINDS]
  bool ready = false;
  // a large prefill runs as two halves on these streams (default priority),
  // forked from and joined back into the caller's stream by the events
  hipStream_t side[2] = {nullptr, nullptr};
  hipEvent_t fork = nullptr, join[2] = {nullptr, nullptr};
  // two-stream split thresholds (allie_model_set_split_tokens; 0: never)
  int tree_heads = 0;  // heads per tree-attention workgroup (allie_model_set_tree_heads; 0: automatic)
  int64_t split_tokens = 24576;  // a prefill's tokens, an extend's tokens
  int64_t split_decode = 512;    // an extend's one-token groups (decode steps)
};

namespace {

// Carves the weight arena (base may be null to size it).
size_t layout_weights(allie_model* m, char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  };
  const size_t d = m->d, V = m->V;
  m->wte = (float*)take(V * d * 4);
  m->wpe = (float*)take((size_t)m->cfg.n_positions * d * 4);
  m->ctrl = (float*)take(2 * d * 4);
  m->lnf_g = (float*)take(d * 4);
  m->lnf_b = (float*)take(d * 4);
  m->w_head = take((size_t)m->NH * d * m->hsz);
  m->b_head = (float*)take((size_t)m->NH * 4);
  m->layers.resize(m->L);
  const bool fp8 = m->cfg.mode == ALLIE_MODE_FP8W;
  for (auto& l : m->layers) {
    l.ln1_g = (float*)take(d * 4);
    l.ln1_b = (float*)take(d * 4);
    l.ln2_g = (float*)take(d * 4);
    l.ln2_b = (float*)take(d * 4);
    l.w_qkv = take(3 * d * d * m->wsz);
    l.b_qkv = (float*)take(3 * d * 4);
    l.w_o = take(d * d * m->wsz);
    l.b_o = (float*)take(d * 4);
    l.w_fc = take(4 * d * d * m->wsz);
    l.b_fc = (float*)take(4 * d * 4);
    l.w_pr = take(4 * d * d * m->wsz);
    l.b_pr = (float*)take(d * 4);
    l.s_qkv = fp8 ? (float*)take(3 * d * 4) : nullptr;
    l.s_o = fp8 ? (float*)take(d * 4) : nullptr;
    l.s_fc = fp8 ? (float*)take(4 * d * 4) : nullptr;
    l.s_pr = fp8 ? (float*)take(d * 4) : nullptr;
  }
  return off;
}

// Uploads n int32 from pageable host memory to dst on stream st without
// synchronising the stream (see PinnedRing).  Not thread-safe per model.
int upload_i32(allie_model* m, int32_t* dst, const int32_t* host, size_t n, hipStream_t st) {
  PinnedRing& r = m->pinned;
  const int i = r.next;
  r.next = (r.next + 1) % PinnedRing::N;
  if (r.used[i]) HIP_TRY(hipEventSynchronize(r.ev[i]));  // its previous upload has been consumed
  if (r.cap[i] < n) {
    if (r.buf[i]) HIP_TRY(hipHostFree(r.buf[i]));
    r.buf[i] = nullptr;
    r.cap[i] = 0;
    const size_t cap = n < 4096 ? 4096 : n * 2;
    HIP_TRY(hipHostMalloc((void**)&r.buf[i], cap * 4, hipHostMallocDefault));
    r.cap[i] = cap;
  }
  if (!r.ev[i]) HIP_TRY(hipEventCreateWithFlags(&r.ev[i], hipEventDisableTiming));
  memcpy(r.buf[i], host, n * 4);
  HIP_TRY(hipMemcpyAsync(dst, r.buf[i], n * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipEventRecord(r.ev[i], st));
  r.used[i] = true;
  return ALLIE_OK;
}

int check_ready(const allie_model* m) {
  if (!m) return fail(ALLIE_ERR_ARG, "model is NULL");
  if (!m->ready) return fail(ALLIE_ERR_STATE, "model not finalised (allie_model_finalize)");
  return ALLIE_OK;
}

bool is_layer_kind(int kind) { return kind >= ALLIE_W_LN1_G && kind <= ALLIE_W_PR_B; }

// fp32 partial sums of the K-split GEMMs of a forward over T token rows
// whose heads run over heads_rows rows (small M only; 0 when none splits).
size_t part_bytes(const allie_model* m, int T, int heads_rows) {
  if (!m->act_bf16) return 0;
  const int d = m->d;
  size_t mx = 0;
  auto need = [&](int M, int N, int K) {
    const int s = gemm_split_factor(M, N, K);
    const size_t b = s > 1 ? (size_t)s * M * N * 4 : 0;
    mx = b > mx ? b : mx;
  };
  need(T, 3 * d, d);
  need(T, d, d);
  need(T, 4 * d, d);
  need(T, d, 4 * d);
  need(heads_rows, m->NH, d);
  // a prefill's last block on the games' last rows
  need(heads_rows, d, d);
  need(heads_rows, 4 * d, d);
  need(heads_rows, d, 4 * d);
  return mx;
}

// Workspace of a prefill of B games / T tokens.
struct PrefillWS {
  int32_t *lens, *cu, *ids, *pos, *seq_of, *last, *blk_off, *tiles, *status, *slot, *order;
  int64_t* in_off;
  float* h;
  void *x, *qkv, *attn, *ff, *hx, *wdq;
  float *z, *part;
  size_t total;
};

// bf16 copy of one layer's largest fp8 weight (4 d^2), fp8-weight models only
size_t wdq_bytes(const allie_model* m) {
  return m->cfg.mode == ALLIE_MODE_FP8W ? (size_t)4 * m->d * m->d * 2 : 0;
}

PrefillWS layout_prefill(const allie_model* m, int B, int T, char* base) {
  PrefillWS w{};
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  };
  const size_t d = m->d, a = m->act_bf16 ? 2 : 4;
  const int max_tiles = (m->cfg.max_length + ATTN_Q_TILE - 1) / ATTN_Q_TILE;
  w.lens = (int32_t*)take((size_t)B * 4);
  w.cu = (int32_t*)take((size_t)(B + 1) * 4);
  w.in_off = (int64_t*)take((size_t)B * 8);
  w.ids = (int32_t*)take((size_t)T * 4);
  w.pos = (int32_t*)take((size_t)T * 4);
  w.seq_of = (int32_t*)take((size_t)T * 4);
  w.slot = (int32_t*)take((size_t)T * 4);
  w.last = (int32_t*)take((size_t)B * 4);
  w.blk_off = (int32_t*)take((size_t)(B + 1) * 4);
  w.tiles = (int32_t*)take((size_t)B * max_tiles * 4);
  w.order = (int32_t*)take((size_t)B * 4);
  w.status = (int32_t*)take(4);
  w.h = (float*)take((size_t)T * d * 4);
  w.x = take((size_t)T * d * a);
  w.qkv = take((size_t)T * 3 * d * a);
  w.attn = take((size_t)T * d * a);
  w.ff = take((size_t)T * 4 * d * a);
  w.hx = take((size_t)B * d * a);
  w.z = (float*)take((size_t)B * m->NH * 4);
  w.part = (float*)take(part_bytes(m, T, B));
  w.wdq = take(wdq_bytes(m));
  w.total = off;
  return w;
}

// part: workspace of the K-split partial sums (part_bytes), or null
// wdq: [4 d^2] bf16 workspace for fp8 weights on the persistent kernel, or null
// Keys and values of an extend's QKV projection written straight to the KV
// pool (layer `layer`, row m at slot[m]) by the GEMM when it can
struct KVDest {
  void* pool;
  const int32_t* slot;
  int layer, pool_blocks;
};

// A skinny GEMM's A operand as the LayerNorm of rows of h (GemmArgs::ln_h)
struct LNSrc {
  const float* h;
  const int32_t* row;  // gather (row m is h row row[m]) or null
  const float* g;
  const float* b;
};

int wtype_of(const allie_model* m) {
  return m->cfg.mode == ALLIE_MODE_FP32 ? W_F32 : (m->cfg.mode == ALLIE_MODE_FP8W ? W_FP8 : W_BF16);
}

// Whether the M x N x K projection of this model after a LayerNorm takes that
// LayerNorm in its prologue (the skinny kernel, bf16 activations): then the
// LayerNorm kernel is not launched and the projection reads h instead of x.
bool ln_fused(const allie_model* m, int M, int N, int K, int wtype) {
  return m->act_bf16 && gemm_skinny_ln_ok(M, N, K, wtype);
}

int gemm(const allie_model* m, const void* A, const void* W, const float* bias, const float* scale,
         void* C, float* R, int M, int N, int K, int epi, int probe_kind, float* part, void* wdq, hipStream_t st,
         const KVDest* kv = nullptr, bool* kv_done = nullptr, const LNSrc* ln = nullptr) {
  GemmArgs g{};
  g.A = A;
  g.W = W;
  g.bias = bias;
  g.scale = scale;
  g.C = C;
  g.R = R;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldc = N;
  g.ldr = N;
  g.epi = epi;
  g.wtype = wtype_of(m);
  g.out_f32 = m->cfg.mode == ALLIE_MODE_FP32;
  g.split = (part && g.wtype != W_F32) ? gemm_split_factor(M, N, K) : 1;
  g.part = part;
  g.wdq = g.wtype == W_FP8 ? wdq : nullptr;
  if (ln) {
    g.ln_h = ln->h;
    g.ln_row = ln->row;
    g.ln_g = ln->g;
    g.ln_b = ln->b;
    g.ln_eps = m->cfg.eps;
  }
  if (kv) {
    g.kv_pool = kv->pool;
    g.kv_slot = kv->slot;
    g.kv_layer = kv->layer;
    g.kv_pool_blocks = kv->pool_blocks;
    if (!gemm_stores_kv(g)) g.kv_pool = nullptr, g.kv_slot = nullptr;
  }
  if (kv_done) *kv_done = g.kv_pool != nullptr;
  HIP_TRY(probe_mark(probe_kind, true, st));
  hipError_t e = launch_gemm(g, st);
  if (e != hipSuccess) return fail(ALLIE_ERR_HIP, "gemm M=%d N=%d K=%d: %s", M, N, K, hipGetErrorString(e));
  HIP_TRY(probe_mark(probe_kind, false, st));
  return ALLIE_OK;
}

// Activations of one forward over T token rows.
struct Acts {
  float* h;   // [T][d] residual stream (fp32)
  void* x;    // [T][d] LayerNorm output
  void* qkv;  // [T][3d]
  void* attn; // [T][d]
  void* ff;   // [T][4d]
  float* part;  // K-split partial sums (part_bytes)
  void* wdq;    // fp8 weights widened to bf16 for the persistent GEMM (wdq_bytes), or null
};

// Whether the M x N x K store GEMM of this model runs on the persistent
// kernel (see gemm()): then the projection feeding the residual stream is
// stored as bf16 and added in the LayerNorm that follows.
bool store_is_persistent(const allie_model* m, int M, int N, int K, const float* part, void* wdq) {
  GemmArgs g{};
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldc = N;
  g.epi = EPI_STORE;
  g.wtype = m->cfg.mode == ALLIE_MODE_FP32 ? W_F32 : (m->cfg.mode == ALLIE_MODE_FP8W ? W_FP8 : W_BF16);
  g.out_f32 = m->cfg.mode == ALLIE_MODE_FP32;
  g.split = (part && g.wtype != W_F32) ? gemm_split_factor(M, N, K) : 1;
  g.wdq = g.wtype == W_FP8 ? wdq : nullptr;
  return gemm_uses_persistent(g);
}

// Rows the last block is finished on when only some rows' outputs are read
// (the heads of a prefill read each game's last token): the last block's
// attention runs over all rows (its keys and values are every row's), then
// its output rows idx[0..n) and their residual rows move into these compact
// buffers and the rest of the block (c_proj, ln_2, MLP) runs on n rows.
struct Compact {
  const int32_t* idx;
  int n;
  void* attn;  // [n][d] activations
  void* x;     // [n][d]
  float* h;    // [n][d] fp32
  void* ff;    // [n][4d]
};

// The transformer blocks over T rows whose embeddings (h) and first ln_1 (x)
// are in place.  kv_slot/kv_pool: every layer's keys and values of row t are
// written to pool slot kv_slot[t] (before attention runs); with kv_only_pool
// the QKV GEMM may write them there instead of into acts.qkv (whose key and
// value columns are then left unwritten: the attention reads them from the
// pool).  attn(layer) runs the attention of one layer from acts.qkv into
// acts.attn.
//
// The attention and MLP output projections end in the residual add
// h += bf16(y + b) (src/modeling/model.py:50-55 -> [lib] GPT2Block).  Small-M
// GEMMs add into h in their epilogue; GEMMs on the persistent kernel store y
// (bf16, into x) and the next LayerNorm adds it (h += y; x = LN(h)).  After
// the last block, *h_final is the residual stream the heads read (acts.h, or
// cp->h when cp finishes the last block on cp->n rows) and *final_add the y
// still to be added to it (the heads' ln_f adds it on the rows it reads), or
// null.
template <typename AttnFn>
int run_layers(const allie_model* m, const Acts& w, int T, const int32_t* kv_slot, void* kv_pool,
               int kv_pool_blocks, bool kv_only_pool, AttnFn&& attn, hipStream_t st, const Compact* cp,
               const float** h_final, const void** final_add) {
  const int d = m->d, L = m->L, act = m->act_bf16;
  *final_add = nullptr;
  *h_final = w.h;
  int rc;
  // the next layer's ln_1 is left to its QKV projection's prologue (the
  // first layer's is fused into the embedding)
  bool ln1_in_qkv = false;
  // c_proj, ln_2 and the MLP of layer li over M rows (attention output in
  // attn, residual stream h), then the next layer's ln_1 into x
  auto finish = [&](int li, int M, void* attn_in, void* x, float* h, void* ff) -> int {
    const LayerW& l = m->layers[li];
    const bool fuse_proj = store_is_persistent(m, M, d, d, w.part, w.wdq);
    const bool fuse_fc2 = store_is_persistent(m, M, d, 4 * d, w.part, w.wdq);
    LNArgs ln{};
    ln.h = h;
    ln.rows = ln.rows_out = M;
    ln.d = d;
    ln.eps = m->cfg.eps;
    ln.y = x;
    ln.act_bf16 = act;
    // With both projections stored as bf16 and a next layer, the attention
    // projection's y goes to the qkv buffer (free once attention has read it)
    // and reaches h only in the next ln_1, with the MLP's: ln_2 normalises
    // h + y_attn without writing h back (8 instead of 12 bytes per element),
    // and ln_1 writes (h + y_attn) + y_mlp, the reference's order of the adds.
    const bool defer = fuse_proj && fuse_fc2 && li + 1 < L && x == w.x;
    void* y_attn = defer ? w.qkv : x;
    int r;
    if (fuse_proj) {
      if ((r = gemm(m, attn_in, l.w_o, l.b_o, l.s_o, y_attn, nullptr, M, d, d, EPI_STORE, ALLIE_PROBE_PROJ, w.part, w.wdq, st))) return r;
    } else {
      if ((r = gemm(m, attn_in, l.w_o, l.b_o, l.s_o, nullptr, h, M, d, d, EPI_RESID, ALLIE_PROBE_PROJ, w.part, w.wdq, st))) return r;
    }
    ln.g = l.ln2_g;
    ln.b = l.ln2_b;
    ln.add = fuse_proj ? y_attn : nullptr;
    ln.h_out = (fuse_proj && !defer) ? h : nullptr;
    // a plain ln_2 (the residual add already in h) before a skinny c_fc runs
    // in that GEMM's prologue
    const LNSrc ln2{h, nullptr, l.ln2_g, l.ln2_b};
    const bool ln2_in_fc = !fuse_proj && ln_fused(m, M, 4 * d, d, wtype_of(m));
    if (!ln2_in_fc) HIP_TRY(launch_layernorm(ln, st));
    if ((r = gemm(m, x, l.w_fc, l.b_fc, l.s_fc, ff, nullptr, M, 4 * d, d, EPI_GELU, ALLIE_PROBE_FC, w.part, w.wdq, st,
                  nullptr, nullptr, ln2_in_fc ? &ln2 : nullptr)))
      return r;
    if (fuse_fc2) {
      if ((r = gemm(m, ff, l.w_pr, l.b_pr, l.s_pr, x, nullptr, M, d, 4 * d, EPI_STORE, ALLIE_PROBE_FC2, w.part, w.wdq, st))) return r;
    } else {
      if ((r = gemm(m, ff, l.w_pr, l.b_pr, l.s_pr, nullptr, h, M, d, 4 * d, EPI_RESID, ALLIE_PROBE_FC2, w.part, w.wdq, st))) return r;
    }
    if (li + 1 < L) {
      ln.g = m->layers[li + 1].ln1_g;
      ln.b = m->layers[li + 1].ln1_b;
      ln.add = fuse_fc2 ? (defer ? y_attn : x) : nullptr;
      ln.add2 = defer ? x : nullptr;
      ln.h_out = fuse_fc2 ? h : nullptr;
      // likewise a plain ln_1 before a skinny QKV projection
      ln1_in_qkv = !fuse_fc2 && ln_fused(m, M, 3 * d, d, wtype_of(m));
      if (!ln1_in_qkv) HIP_TRY(launch_layernorm(ln, st));
    } else {
      *final_add = fuse_fc2 ? x : nullptr;
    }
    return ALLIE_OK;
  };
  for (int li = 0; li < L; ++li) {
    const LayerW& l = m->layers[li];
    const KVDest kvd{kv_pool, kv_slot, li, kv_pool_blocks};
    bool kv_done = false;
    const LNSrc ln1{w.h, nullptr, l.ln1_g, l.ln1_b};
    if ((rc = gemm(m, w.x, l.w_qkv, l.b_qkv, l.s_qkv, w.qkv, nullptr, T, 3 * d, d, EPI_STORE, ALLIE_PROBE_QKV, w.part,
                   w.wdq, st, (kv_only_pool && kv_pool && kv_slot) ? &kvd : nullptr, &kv_done,
                   ln1_in_qkv ? &ln1 : nullptr)))
      return rc;
    ln1_in_qkv = false;
    if (kv_pool && kv_slot && !kv_done) {
      KVWriteArgs kw{};
      kw.qkv = w.qkv;
      kw.slot = kv_slot;
      kw.T = T;
      kw.n_layer = L;
      kw.layer = li;
      kw.n_head = m->H;
      kw.head_dim = m->hd;
      kw.pool_blocks = kv_pool_blocks;
      kw.pool = kv_pool;
      kw.act_bf16 = act;
      HIP_TRY(launch_kv_write(kw, st));
    }
    if ((rc = attn(li))) return rc;
    if (li + 1 == L && cp) {
      // the residual stream is current here: the last ln_1 wrote back its add
      const int a = act ? 2 : 4;
      HIP_TRY(launch_gather_rows(w.attn, cp->idx, cp->n, d * a, cp->attn, st));
      HIP_TRY(launch_gather_rows(w.h, cp->idx, cp->n, d * 4, cp->h, st));
      *h_final = cp->h;
      return finish(li, cp->n, cp->attn, cp->x, cp->h, cp->ff);
    }
    if ((rc = finish(li, T, w.attn, w.x, w.h, w.ff))) return rc;
  }
  return ALLIE_OK;
}

// ln_f, the heads GEMM and the heads kernel over `rows` rows of h (row r is
// h[row_idx[r]], or h[r] when row_idx is null; plus h_add's row when the last
// block's residual add is still pending); hx [rows][d] and z [rows][NH] are
// scratch.
int run_heads(const allie_model* m, const float* h, const void* h_add, const int32_t* row_idx, int rows, void* hx,
              float* z, float temperature, const uint32_t* legal, int legal_words, const allie_outputs* out,
              float* part, hipStream_t st) {
  const int d = m->d, act = m->act_bf16;
  LNArgs lf{};
  lf.h = h;
  lf.add = h_add;
  lf.row_idx = row_idx;
  lf.rows = lf.rows_out = rows;
  lf.d = d;
  lf.g = m->lnf_g;
  lf.b = m->lnf_b;
  lf.eps = m->cfg.eps;
  lf.y = hx;
  lf.act_bf16 = act;
  // ln_f in the heads GEMM's prologue when that GEMM is skinny and no
  // residual add is pending
  const bool lnf_in_gemm = !h_add && ln_fused(m, rows, m->NH, d, W_BF16);
  if (!lnf_in_gemm) HIP_TRY(launch_layernorm(lf, st));
  {
    GemmArgs g{};
    if (lnf_in_gemm) {
      g.ln_h = h;
      g.ln_row = row_idx;
      g.ln_g = m->lnf_g;
      g.ln_b = m->lnf_b;
      g.ln_eps = m->cfg.eps;
    }
    g.A = hx;
    g.W = m->w_head;
    g.bias = m->b_head;
    g.C = z;
    g.M = rows;
    g.N = m->NH;
    g.K = d;
    g.lda = d;
    g.ldc = m->NH;
    g.epi = EPI_STORE;
    g.wtype = act ? W_BF16 : W_F32;
    g.out_f32 = 1;
    g.split = (part && act) ? gemm_split_factor(rows, g.N, d) : 1;
    g.part = part;
    hipError_t e = launch_gemm(g, st);
    if (e != hipSuccess) return fail(ALLIE_ERR_HIP, "heads gemm: %s", hipGetErrorString(e));
  }
  HeadsArgs ha{};
  ha.z = z;
  ha.B = rows;
  ha.ldz = m->NH;
  ha.vocab = m->V;
  ha.n_moves = 1968;
  ha.value_col = m->V;
  ha.time_col = m->V + 1;
  ha.temperature = temperature > 1e-5f ? temperature : 1e-5f;
  ha.legal = legal;
  ha.legal_words = legal_words;
  ha.logits = out->logits;
  ha.logits_raw = out->logits_raw;
  ha.value = out->value;
  ha.time = out->time;
  ha.top1 = out->top1;
  ha.lse = out->lse;
  ha.max_logit = out->max_logit;
  ha.emulate_bf16 = act;
  HIP_TRY(launch_heads(ha, st));
  return ALLIE_OK;
}

// Workspace of an extend of n tokens in G groups.
struct ExtendWS {
  int32_t *group_start, *tiles, *self_slot, *status, *order;
  float* h;
  void *x, *qkv, *attn, *ff, *hx, *wdq;
  float *z, *part;
  size_t total;
};

// with_wdq: include the fp8 widening buffer (only large-M GEMMs use it)
ExtendWS layout_extend(const allie_model* m, int n, int G, char* base, bool with_wdq) {
  ExtendWS w{};
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  };
  const size_t d = m->d, a = m->act_bf16 ? 2 : 4;
  w.group_start = (int32_t*)take((size_t)(G + 1) * 4);
  w.tiles = (int32_t*)take(((size_t)n / 64 + G + 1) * 4);  // >= sum of ceil(size / 64)
  w.self_slot = (int32_t*)take((size_t)n * 4);
  w.status = (int32_t*)take(4);
  w.order = (int32_t*)take((size_t)n * 4);
  w.h = (float*)take((size_t)n * d * 4);
  w.x = take((size_t)n * d * a);
  w.qkv = take((size_t)n * 3 * d * a);
  w.attn = take((size_t)n * d * a);
  w.ff = take((size_t)n * 4 * d * a);
  w.hx = take((size_t)n * d * a);
  w.z = (float*)take((size_t)n * m->NH * 4);
  w.part = (float*)take(part_bytes(m, n, n));
  w.wdq = with_wdq ? take(wdq_bytes(m)) : nullptr;
  w.total = off;
  return w;
}

// A bf16 prefill of at least m->split_tokens tokens (and no KV pool or
// status output) runs as two halves on two streams; so does an extend of as
// many tokens, or of at least m->split_decode one-token groups (decode steps)
bool split_size(const allie_model* m, int64_t tokens) {
  return m->act_bf16 && m->split_tokens > 0 && tokens >= m->split_tokens;
}
bool split_decode_size(const allie_model* m, int64_t one_token_groups) {
  return m->act_bf16 && m->split_decode > 0 && one_token_groups >= m->split_decode;
}

// *out = *a | *b (the validation flags of an extend's two halves)
__global__ void or_status_kernel(int32_t* out, const int32_t* a, const int32_t* b) {
  if (threadIdx.x == 0) *out = *a | *b;
}

// One prefill forward of n_seq games (T tokens) over the laid-out workspace
// w, on stream st (arguments checked by allie_prefill).
int prefill_batch(allie_model* m, const uint32_t* words, const int32_t* lens_host, int n_seq, int64_t T,
                  float temperature, const uint32_t* legal, int legal_words, const allie_outputs* out,
                  void* kv_pool, int kv_pool_blocks, int first_block, const int32_t* kv_block_table,
                  int kv_max_blocks, int32_t* status, const PrefillWS& w, hipStream_t st) {
  int rc;
  const int d = m->d, L = m->L, act = m->act_bf16;
  const int max_len = m->cfg.max_length;
  int64_t n_tiles = 0;
  for (int i = 0; i < n_seq; ++i) {
    const int n = lens_host[i] < max_len ? lens_host[i] : max_len;
    n_tiles += (n + ATTN_Q_TILE - 1) / ATTN_Q_TILE;
  }
  const float eps = m->cfg.eps;

  if ((rc = upload_i32(m, w.lens, lens_host, (size_t)n_seq, st))) return rc;
  PackArgs p{};
  p.words = words;
  p.lens = w.lens;
  p.B = n_seq;
  p.max_len = max_len;
  p.block = KV_BLOCK;
  p.first_block = first_block;
  p.max_blocks = (max_len + KV_BLOCK - 1) / KV_BLOCK;
  p.q_tile = ATTN_Q_TILE;
  p.capacity = (int)T;
  p.cu_seqlens = w.cu;
  p.in_off = w.in_off;
  p.ids = w.ids;
  p.pos = w.pos;
  p.seq_of = w.seq_of;
  p.last_idx = w.last;
  p.blk_off = w.blk_off;
  p.block_table = nullptr;
  p.slot = kv_pool ? w.slot : nullptr;
  p.tiles = w.tiles;
  p.block_table_in = kv_block_table;
  p.max_blocks_in = kv_max_blocks;
  p.pad_id = ALLIE_PAD_ID;
  p.status = status ? status : w.status;
  HIP_TRY(launch_pack(p, st));

  EmbedArgs ea{};
  ea.ids = w.ids;
  ea.pos = w.pos;
  ea.T = (int)T;
  ea.d = d;
  ea.vocab = m->V;
  ea.n_positions = m->cfg.n_positions;
  ea.wte = m->wte;
  ea.wpe = m->wpe;
  ea.ctrl = m->ctrl;
  ea.ln_g = m->layers[0].ln1_g;
  ea.ln_b = m->layers[0].ln1_b;
  ea.eps = eps;
  ea.h = w.h;
  ea.x = w.x;
  ea.act_bf16 = act;
  HIP_TRY(launch_embed_ln(ea, st));

  AttnVarlenArgs aa{};
  aa.qkv = w.qkv;
  aa.cu_seqlens = w.cu;
  aa.tiles = w.tiles;
  aa.n_tiles = (int)n_tiles;
  aa.order = w.order;
  aa.B = n_seq;
  aa.T = (int)T;
  aa.n_head = m->H;
  aa.head_dim = m->hd;
  aa.scale = 0.125f;  // 1 / sqrt(64)
  aa.out = w.attn;
  aa.act_bf16 = act;

  const Acts acts{w.h, w.x, w.qkv, w.attn, w.ff, w.part, w.wdq};
  // Only each game's last token reaches the heads, so the last block's c_proj,
  // ln_2 and MLP run on those n_seq rows (when they are at most half the
  // tokens): its attention output and residual rows are gathered into x
  // (free once the block's QKV has read it) and ff (not yet written).
  Compact cp{};
  const bool compact = 2 * (int64_t)n_seq <= T;
  if (compact) {
    const size_t a = act ? 2 : 4;
    cp.idx = w.last;
    cp.n = n_seq;
    cp.attn = w.x;
    cp.x = (char*)w.x + align_up((size_t)n_seq * d * a);
    cp.h = (float*)w.ff;
    cp.ff = (char*)w.ff + align_up((size_t)n_seq * d * 4);
  }
  const void* final_add = nullptr;
  const float* h_final = nullptr;
  rc = run_layers(m, acts, (int)T, kv_pool ? w.slot : nullptr, kv_pool, kv_pool_blocks, false,
                  [&](int layer) -> int {
                    HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, true, st));
                    aa.order_ready = layer > 0;  // the game order is computed once per forward
                    aa.last_only = compact && layer == L - 1;  // only the compact rows are read
                    HIP_TRY(launch_attn_varlen(aa, st));
                    HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, false, st));
                    return ALLIE_OK;
                  },
                  st, compact ? &cp : nullptr, &h_final, &final_add);
  if (rc) return rc;
  // heads on the last token of every game (row b of the compact rows is game b's)
  return run_heads(m, h_final, final_add, compact ? nullptr : w.last, n_seq, w.hx, w.z, temperature, legal,
                   legal_words, out, w.part, st);
}


}  // namespace

extern "C" {

const char* allie_last_error(void) { return g_err.c_str(); }
int allie_abi_version(void) { return 1; }

int allie_model_create(const allie_config* cfg, allie_model** out) {
  if (!cfg || !out) return fail(ALLIE_ERR_ARG, "NULL argument");
  *out = nullptr;
  if (cfg->n_layer <= 0 || cfg->d_model <= 0 || cfg->n_head <= 0 || cfg->vocab_size <= 2)
    return fail(ALLIE_ERR_ARG, "bad config");
  if (cfg->d_model % cfg->n_head != 0 || cfg->d_model / cfg->n_head != 64)
    return fail(ALLIE_ERR_ARG, "head_dim must be 64 (d_model %d, n_head %d)", cfg->d_model, cfg->n_head);
  if (cfg->d_model % 256 != 0 || cfg->d_model > 2048)
    return fail(ALLIE_ERR_ARG, "d_model must be a multiple of 256 and <= 2048");
  if (cfg->max_length <= 0 || cfg->max_length > 512 || cfg->max_length > cfg->n_positions)
    return fail(ALLIE_ERR_ARG, "max_length must be in [1, min(512, n_positions)]");
  if (cfg->mode < ALLIE_MODE_FP32 || cfg->mode > ALLIE_MODE_FP8W) return fail(ALLIE_ERR_ARG, "bad mode");
  int dev = 0;
  hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return fail(ALLIE_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(de));
  // address of this device's copy of the allocation-free scratch
  de = scratch_init(dev);
  if (de != hipSuccess)
    return fail(ALLIE_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(de));
  allie_model* m = new allie_model();
  m->cfg = *cfg;
  m->device = dev;
  m->d = cfg->d_model;
  m->H = cfg->n_head;
  m->hd = 64;
  m->L = cfg->n_layer;
  m->V = cfg->vocab_size;
  m->NH = (m->V + 2 + 255) / 256 * 256;
  m->wsz = cfg->mode == ALLIE_MODE_FP32 ? 4 : (cfg->mode == ALLIE_MODE_FP8W ? 1 : 2);
  m->hsz = cfg->mode == ALLIE_MODE_FP32 ? 4 : 2;
  m->act_bf16 = cfg->mode != ALLIE_MODE_FP32;
  m->arena_bytes = layout_weights(m, nullptr);
  hipError_t e = hipMalloc((void**)&m->arena, m->arena_bytes);
  if (e != hipSuccess) {
    const size_t m_bytes = m->arena_bytes;
    delete m;
    return fail(ALLIE_ERR_NOMEM, "hipMalloc(%zu): %s", m_bytes, hipGetErrorString(e));
  }
  layout_weights(m, m->arena);
  // zero padding rows of the heads matrix and unset biases
  e = hipMemset(m->arena, 0, m->arena_bytes);
  if (e != hipSuccess) {
    (void)hipFree(m->arena);
    delete m;
    return fail(ALLIE_ERR_HIP, "hipMemset: %s", hipGetErrorString(e));
  }
  m->set.assign((size_t)(m->L + 1) * N_KINDS, 0);
  // the two streams of a split prefill and their fork / join events
  if (m->act_bf16) {
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
      e = hipStreamCreateWithFlags(&m->side[i], hipStreamNonBlocking);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&m->join[i], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->fork, hipEventDisableTiming);
    if (e != hipSuccess) {
      allie_model_destroy(m);
      return fail(ALLIE_ERR_HIP, "stream / event creation: %s", hipGetErrorString(e));
    }
  }
  *out = m;
  return ALLIE_OK;
}

void allie_model_destroy(allie_model* m) {
  if (!m) return;
  // teardown: a failing release has no caller to report to, so results are
  // not checked here
  for (int i = 0; i < 2; ++i) {
    if (m->side[i]) {
      (void)hipStreamSynchronize(m->side[i]);
      (void)hipStreamDestroy(m->side[i]);
    }
    if (m->join[i]) (void)hipEventDestroy(m->join[i]);
  }
  if (m->fork) (void)hipEventDestroy(m->fork);
  for (int i = 0; i < PinnedRing::N; ++i) {
    if (m->pinned.ev[i]) {
      (void)hipEventSynchronize(m->pinned.ev[i]);
      (void)hipEventDestroy(m->pinned.ev[i]);
    }
    if (m->pinned.buf[i]) (void)hipHostFree(m->pinned.buf[i]);
  }
  if (m->arena) (void)hipFree(m->arena);
  delete m;
}

int allie_model_set_weight(allie_model* m, int kind, int layer, const float* src, int64_t rows,
                           int64_t cols, void* stream) {
  if (!m || !src) return fail(ALLIE_ERR_ARG, "NULL argument");
  hipStream_t st = (hipStream_t)stream;
  const int64_t d = m->d, V = m->V;
  const int rb = m->act_bf16;  // bf16 modes round biases to bf16 (autocast addmm)
  const int hb = m->hsz == 2;
  auto want = [&](int64_t r, int64_t c) -> bool { return rows == r && cols == c; };
  auto bad_shape = [&]() {
    return fail(ALLIE_ERR_ARG, "weight kind %d: unexpected shape %lld x %lld", kind, (long long)rows,
                (long long)cols);
  };
  if (is_layer_kind(kind)) {
    if (layer < 0 || layer >= m->L) return fail(ALLIE_ERR_ARG, "layer %d out of range", layer);
    LayerW& l = m->layers[layer];
    const bool fp8 = m->cfg.mode == ALLIE_MODE_FP8W;
    switch (kind) {
      case ALLIE_W_LN1_G: case ALLIE_W_LN1_B: case ALLIE_W_LN2_G: case ALLIE_W_LN2_B: {
        if (rows * cols != d) return bad_shape();
        float* dst = kind == ALLIE_W_LN1_G ? l.ln1_g : kind == ALLIE_W_LN1_B ? l.ln1_b
                   : kind == ALLIE_W_LN2_G ? l.ln2_g : l.ln2_b;
        HIP_TRY(hipMemcpyAsync(dst, src, d * 4, hipMemcpyDeviceToDevice, st));
        break;
      }
      case ALLIE_W_QKV_B: case ALLIE_W_O_B: case ALLIE_W_FC_B: case ALLIE_W_PR_B: {
        const int64_t n = kind == ALLIE_W_QKV_B ? 3 * d : kind == ALLIE_W_FC_B ? 4 * d : d;
        if (rows * cols != n) return bad_shape();
        float* dst = kind == ALLIE_W_QKV_B ? l.b_qkv : kind == ALLIE_W_O_B ? l.b_o
                   : kind == ALLIE_W_FC_B ? l.b_fc : l.b_pr;
        HIP_TRY(launch_convert(src, n, dst, 0, rb, st));
        break;
      }
      case ALLIE_W_QKV_W: case ALLIE_W_O_W: case ALLIE_W_FC_W: case ALLIE_W_PR_W: {
        if (fp8) return fail(ALLIE_ERR_ARG, "fp8 mode: set block GEMM weights with allie_model_set_weight_fp8");
        int64_t in = d, outf = d;
        void* dst = l.w_o;
        if (kind == ALLIE_W_QKV_W) { outf = 3 * d; dst = l.w_qkv; }
        if (kind == ALLIE_W_FC_W) { outf = 4 * d; dst = l.w_fc; }
        if (kind == ALLIE_W_PR_W) { in = 4 * d; dst = l.w_pr; }
        if (!want(in, outf)) return bad_shape();
        HIP_TRY(launch_transpose_convert(src, (int)in, (int)outf, dst, rb, (int)in, st));
        break;
      }
      default: return fail(ALLIE_ERR_ARG, "unknown weight kind %d", kind);
    }
    m->set[(size_t)(layer + 1) * N_KINDS + (kind - ALLIE_W_LN1_G)] = 1;
    return ALLIE_OK;
  }
  switch (kind) {
    case ALLIE_W_WTE:
      if (!want(V, d)) return bad_shape();
      HIP_TRY(hipMemcpyAsync(m->wte, src, V * d * 4, hipMemcpyDeviceToDevice, st));
      HIP_TRY(launch_convert(src, V * d, m->w_head, hb, 0, st));
      break;
    case ALLIE_W_WPE:
      if (!want(m->cfg.n_positions, d)) return bad_shape();
      HIP_TRY(hipMemcpyAsync(m->wpe, src, (size_t)m->cfg.n_positions * d * 4, hipMemcpyDeviceToDevice, st));
      break;
    case ALLIE_W_CTRL:
      if (!want(2, d)) return bad_shape();
      HIP_TRY(hipMemcpyAsync(m->ctrl, src, 2 * d * 4, hipMemcpyDeviceToDevice, st));
      break;
    case ALLIE_W_LNF_G: case ALLIE_W_LNF_B:
      if (rows * cols != d) return bad_shape();
      HIP_TRY(hipMemcpyAsync(kind == ALLIE_W_LNF_G ? m->lnf_g : m->lnf_b, src, d * 4,
                             hipMemcpyDeviceToDevice, st));
      break;
    case ALLIE_W_VALUE_W: case ALLIE_W_TIME_W: {
      if (rows * cols != d) return bad_shape();
      const int64_t row = kind == ALLIE_W_VALUE_W ? V : V + 1;
      char* dst = (char*)m->w_head + row * d * m->hsz;
      HIP_TRY(launch_convert(src, d, dst, hb, 0, st));
      break;
    }
    case ALLIE_W_VALUE_B: case ALLIE_W_TIME_B: {
      if (rows * cols != 1) return bad_shape();
      const int64_t row = kind == ALLIE_W_VALUE_B ? V : V + 1;
      HIP_TRY(launch_convert(src, 1, m->b_head + row, 0, rb, st));
      break;
    }
    default: return fail(ALLIE_ERR_ARG, "unknown weight kind %d", kind);
  }
  m->set[kind] = 1;
  return ALLIE_OK;
}

int allie_model_set_weight_fp8(allie_model* m, int kind, int layer, const uint8_t* q,
                               const float* scale, int64_t out_features, int64_t in_features,
                               void* stream) {
  if (!m || !q || !scale) return fail(ALLIE_ERR_ARG, "NULL argument");
  if (m->cfg.mode != ALLIE_MODE_FP8W) return fail(ALLIE_ERR_ARG, "model is not in fp8 mode");
  if (layer < 0 || layer >= m->L) return fail(ALLIE_ERR_ARG, "layer %d out of range", layer);
  hipStream_t st = (hipStream_t)stream;
  LayerW& l = m->layers[layer];
  const int64_t d = m->d;
  void* dst;
  float* sdst;
  int64_t in = d, outf = d;
  switch (kind) {
    case ALLIE_W_QKV_W: dst = l.w_qkv; sdst = l.s_qkv; outf = 3 * d; break;
    case ALLIE_W_O_W: dst = l.w_o; sdst = l.s_o; break;
    case ALLIE_W_FC_W: dst = l.w_fc; sdst = l.s_fc; outf = 4 * d; break;
    case ALLIE_W_PR_W: dst = l.w_pr; sdst = l.s_pr; in = 4 * d; break;
    default: return fail(ALLIE_ERR_ARG, "fp8 weights are only for the block GEMMs (kind %d)", kind);
  }
  if (out_features != outf || in_features != in)
    return fail(ALLIE_ERR_ARG, "fp8 weight kind %d: unexpected shape %lld x %lld", kind,
                (long long)out_features, (long long)in_features);
  HIP_TRY(hipMemcpyAsync(dst, q, outf * in, hipMemcpyDeviceToDevice, st));
  HIP_TRY(hipMemcpyAsync(sdst, scale, outf * 4, hipMemcpyDeviceToDevice, st));
  m->set[(size_t)(layer + 1) * N_KINDS + (kind - ALLIE_W_LN1_G)] = 1;
  return ALLIE_OK;
}

int allie_model_set_split_tokens(allie_model* m, int64_t tokens, int64_t decode_tokens) {
  if (!m) return fail(ALLIE_ERR_ARG, "null model");
  if (tokens < 0 || decode_tokens < 0)
    return fail(ALLIE_ERR_ARG, "split thresholds %lld, %lld < 0", (long long)tokens, (long long)decode_tokens);
  m->split_tokens = tokens;
  m->split_decode = decode_tokens;
  return ALLIE_OK;
}

int allie_model_set_tree_heads(allie_model* m, int heads) {
  if (!m) return fail(ALLIE_ERR_ARG, "null model");
  if (heads < 0 || heads > 16 || (heads > 0 && m->H % heads != 0))
    return fail(ALLIE_ERR_ARG, "tree heads %d: 0, or a divisor of %d heads up to 16", heads, m->H);
  m->tree_heads = heads;
  return ALLIE_OK;
}

int allie_model_finalize(allie_model* m) {
  if (!m) return fail(ALLIE_ERR_ARG, "model is NULL");
  for (int k = ALLIE_W_WTE; k <= ALLIE_W_TIME_B; ++k)
    if (!m->set[k]) return fail(ALLIE_ERR_STATE, "global weight kind %d not set", k);
  for (int l = 0; l < m->L; ++l)
    for (int k = ALLIE_W_LN1_G; k <= ALLIE_W_PR_B; ++k)
      if (!m->set[(size_t)(l + 1) * N_KINDS + (k - ALLIE_W_LN1_G)])
        return fail(ALLIE_ERR_STATE, "layer %d weight kind %d not set", l, k);
  m->ready = true;
  return ALLIE_OK;
}

int allie_pack_ragged(const uint32_t* words, const int32_t* lens, int n_seq, int max_len,
                      int block, int first_block, int max_blocks, int capacity,
                      int32_t* cu_seqlens, int64_t* in_off, int32_t* ids, int32_t* pos,
                      int32_t* seq_of, int32_t* last_idx, int32_t* blk_off,
                      int32_t* block_table, int32_t* slot, int pad_id, int32_t* status,
                      void* stream) {
  if (n_seq < 0 || max_len <= 0 || block <= 0 || max_blocks < 0 || capacity < 0)
    return fail(ALLIE_ERR_ARG, "bad pack sizes");
  if (!lens || !cu_seqlens || !in_off || !last_idx || !blk_off || !status ||
      (capacity > 0 && (!ids || !pos || !seq_of) ) || (n_seq > 0 && !words))
    return fail(ALLIE_ERR_ARG, "NULL argument");
  PackArgs p{};
  p.words = words;
  p.lens = lens;
  p.B = n_seq;
  p.max_len = max_len;
  p.block = block;
  p.first_block = first_block;
  p.max_blocks = max_blocks;
  p.q_tile = ATTN_Q_TILE;
  p.capacity = capacity;
  p.cu_seqlens = cu_seqlens;
  p.in_off = in_off;
  p.ids = ids;
  p.pos = pos;
  p.seq_of = seq_of;
  p.last_idx = last_idx;
  p.blk_off = blk_off;
  p.block_table = block_table;
  p.slot = slot;
  p.tiles = nullptr;
  p.pad_id = pad_id;
  p.status = status;
  HIP_TRY(launch_pack(p, (hipStream_t)stream));
  return ALLIE_OK;
}

size_t allie_prefill_workspace_bytes(const allie_model* m, int n_seq, int n_tokens) {
  if (!m || n_seq < 0 || n_tokens < 0) return 0;
  size_t b = layout_prefill(m, n_seq, n_tokens, nullptr).total;
  // a prefill that runs as two halves needs a second copy of the per-game
  // and fixed parts and the alignment of the second half's arrays (a smaller
  // workspace runs it in one piece)
  if (split_size(m, n_tokens) && n_seq >= 2)
    b += layout_prefill(m, n_seq, 0, nullptr).total + 32 * 256;
  return b;
}

size_t allie_kv_block_bytes(const allie_model* m) {
  if (!m) return 0;
  return (size_t)m->L * 2 * m->H * KV_BLOCK * m->hd * (m->act_bf16 ? 2 : 4);
}

int allie_prefill(allie_model* m, const uint32_t* words, const int32_t* lens_host, int n_seq,
                  float temperature, const uint32_t* legal, int legal_words,
                  const allie_outputs* out, void* kv_pool, int kv_pool_blocks, int first_block,
                  const int32_t* kv_block_table, int kv_max_blocks, int32_t* status,
                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_ready(m);
  if (rc) return rc;
  if (n_seq <= 0 || !words || !lens_host || !out || !workspace)
    return fail(ALLIE_ERR_ARG, "bad prefill arguments");
  if (!out->value || !out->time || !out->top1 || !out->max_logit || !out->lse)
    return fail(ALLIE_ERR_ARG, "value/time/top1/max_logit/lse outputs are required");
  if (legal && legal_words * 32 < 1968) return fail(ALLIE_ERR_ARG, "legal mask too narrow");
  const int max_len = m->cfg.max_length;
  int64_t T = 0, n_blocks = 0;
  for (int i = 0; i < n_seq; ++i) {
    if (lens_host[i] <= 0) return fail(ALLIE_ERR_LENGTH, "game %d is empty", i);
    const int n = lens_host[i] < max_len ? lens_host[i] : max_len;
    T += n;
    n_blocks += (n + KV_BLOCK - 1) / KV_BLOCK;
  }
  if (T > (int64_t)1 << 30) return fail(ALLIE_ERR_ARG, "too many tokens");
  if (kv_block_table && kv_max_blocks <= 0) return fail(ALLIE_ERR_ARG, "kv_max_blocks must be positive");
  if (kv_pool && !kv_block_table && (first_block < 0 || first_block + n_blocks > kv_pool_blocks))
    return fail(ALLIE_ERR_LENGTH, "KV pool too small: need blocks [%d, %lld), have %d", first_block,
                (long long)(first_block + n_blocks), kv_pool_blocks);
  hipStream_t st = (hipStream_t)stream;
  const PrefillWS w = layout_prefill(m, n_seq, (int)T, (char*)workspace);
  // Large bf16 batches run as two halves of consecutive games, one per side
  // stream: the halves' kernels fill each other's idle resources (a
  // LayerNorm or attention of one half beside the other's persistent GEMM,
  // the GEMMs' last partial rounds).  Rows never interact across games, so
  // each half computes exactly what the whole batch would for its games.
  int cut = 0;
  int64_t T0 = 0;
  if (split_size(m, T) && !kv_pool && !status && n_seq >= 2) {
    int64_t acc = 0;
    for (int i = 0; i < n_seq - 1; ++i) {
      acc += lens_host[i] < max_len ? lens_host[i] : max_len;
      if (2 * acc >= T) {
        cut = i + 1;
        T0 = acc;
        break;
      }
    }
    if (cut == 0) {
      cut = n_seq - 1;
      T0 = acc;
    }
  }
  if (cut > 0) {
    const PrefillWS w0 = layout_prefill(m, cut, (int)T0, (char*)workspace);
    const PrefillWS w1 = layout_prefill(m, n_seq - cut, (int)(T - T0), (char*)workspace + w0.total);
    int dev = -1;
    if (w0.total + w1.total > workspace_bytes || !m->fork || hipGetDevice(&dev) != hipSuccess || dev != m->device)
      cut = 0;
    if (cut > 0) {
      HIP_TRY(hipEventRecord(m->fork, st));
      int64_t words0 = 0;  // the second half's words start after the first half's games
      for (int i = 0; i < cut; ++i) words0 += lens_host[i];
      allie_outputs o1 = *out;
      auto shift = [&](auto* p, int64_t n) { return p ? p + n : p; };
      o1.logits = shift(out->logits, (int64_t)cut * m->V);
      o1.logits_raw = shift(out->logits_raw, (int64_t)cut * m->V);
      o1.value = out->value + cut;
      o1.time = out->time + cut;
      o1.top1 = out->top1 + cut;
      o1.max_logit = out->max_logit + cut;
      o1.lse = out->lse + cut;
      for (int i = 0; i < 2; ++i) {
        HIP_TRY(hipStreamWaitEvent(m->side[i], m->fork, 0));
        rc = i == 0 ? prefill_batch(m, words, lens_host, cut, T0, temperature, legal, legal_words, out, nullptr, 0,
                                    0, nullptr, 0, nullptr, w0, m->side[0])
                    : prefill_batch(m, words + words0, lens_host + cut, n_seq - cut, T - T0, temperature,
                                    legal ? legal + (int64_t)cut * legal_words : nullptr, legal_words, &o1, nullptr,
                                    0, 0, nullptr, 0, nullptr, w1, m->side[1]);
        if (rc) return rc;
        HIP_TRY(hipEventRecord(m->join[i], m->side[i]));
        HIP_TRY(hipStreamWaitEvent(st, m->join[i], 0));
      }
      return ALLIE_OK;
    }
  }
  if (workspace_bytes < w.total)
    return fail(ALLIE_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, w.total);
  return prefill_batch(m, words, lens_host, n_seq, T, temperature, legal, legal_words, out, kv_pool, kv_pool_blocks,
                       first_block, kv_block_table, kv_max_blocks, status, w, st);
}

size_t allie_extend_workspace_bytes(const allie_model* m, int n_tok, int n_groups) {
  if (!m || n_tok < 0 || n_groups < 0) return 0;
  size_t b = layout_extend(m, n_tok, n_groups, nullptr, true).total;
  // room for the two halves of a split extend (see allie_prefill_workspace_bytes)
  if ((split_size(m, n_tok) || split_decode_size(m, n_tok)) && n_groups >= 2)
    b += layout_extend(m, 0, n_groups, nullptr, true).total + 32 * 256;
  return b;
}

}  // extern "C"

namespace {

// Checks an extend batch on the host; fills the plan of which attention
// kernels run (see extend_run).
struct ExtendPlan {
  int n1 = 0;        // leading groups of one token each (decode steps)
  int max_group = 0;
  int max_rest = 0;  // largest group after those
  int tile_q = 64;   // queries per tree-kernel tile
  int64_t n_tiles = 0;
};

int extend_check(const allie_model* m, const int32_t* ids, const int32_t* pos, int n_tok,
                 const int32_t* group_start_host, int n_groups, const int32_t* prefix_len,
                 const int32_t* prefix_blocks, int max_blocks, const int32_t* extra_slot,
                 const int32_t* n_extra, int max_extra, const uint32_t* legal, int legal_words,
                 const allie_outputs* out, void* kv_pool, int kv_pool_blocks, ExtendPlan* plan) {
  int rc = check_ready(m);
  if (rc) return rc;
  if (n_tok <= 0 || n_groups <= 0 || !ids || !pos || !group_start_host || !prefix_len ||
      !extra_slot || !n_extra || !out || !kv_pool || max_extra <= 0 || max_blocks < 0 ||
      (max_blocks > 0 && !prefix_blocks) || kv_pool_blocks <= 0)
    return fail(ALLIE_ERR_ARG, "bad extend arguments");
  if (!out->value || !out->time || !out->top1 || !out->max_logit || !out->lse)
    return fail(ALLIE_ERR_ARG, "value/time/top1/max_logit/lse outputs are required");
  if (legal && legal_words * 32 < 1968) return fail(ALLIE_ERR_ARG, "legal mask too narrow");
  // groups: contiguous, non-empty, covering [0, n_tok)
  if (group_start_host[0] != 0 || group_start_host[n_groups] != n_tok)
    return fail(ALLIE_ERR_ARG, "group_start must run from 0 to n_tok");
  if (n_groups > (1 << 23)) return fail(ALLIE_ERR_ARG, "too many groups");
  ExtendPlan p;
  for (int g = 0; g < n_groups; ++g) {
    const int sz = group_start_host[g + 1] - group_start_host[g];
    if (sz <= 0) return fail(ALLIE_ERR_ARG, "group %d is empty", g);
    if (sz > 64 * 256) return fail(ALLIE_ERR_ARG, "group %d has %d tokens (max 16384)", g, sz);
    p.max_group = sz > p.max_group ? sz : p.max_group;
    if (p.n1 == g && sz == 1) p.n1 = g + 1;
    if (g >= p.n1) p.max_rest = sz > p.max_rest ? sz : p.max_rest;
  }
  // queries per tree-kernel tile: 128 when some group is larger than 64
  p.tile_q = p.max_rest > 64 ? 128 : 64;
  // the tree and fan kernels (bf16 modes only; the fp32 check mode runs every
  // group on the wave kernel, which takes any table width) stage the table
  if (m->act_bf16 && p.max_rest > FAN_MAX_Q && max_blocks > TREE_MAX_BLOCKS)
    return fail(ALLIE_ERR_ARG, "groups of more than %d tokens take block tables of at most %d blocks (got %d)",
                FAN_MAX_Q, TREE_MAX_BLOCKS, max_blocks);
  if (m->act_bf16 && p.max_rest > 1 && max_blocks > FAN_MAX_BLOCKS)
    return fail(ALLIE_ERR_ARG, "groups of several tokens take block tables of at most %d blocks (got %d)",
                FAN_MAX_BLOCKS, max_blocks);
  for (int g = p.n1; g < n_groups; ++g)
    p.n_tiles += (group_start_host[g + 1] - group_start_host[g] + p.tile_q - 1) / p.tile_q;
  *plan = p;
  return ALLIE_OK;
}

// The extend forward over a laid-out workspace w whose w.group_start already
// holds the group starts on the device (or group_start_dev, when given).
int extend_run(allie_model* m, const ExtendPlan& plan, const ExtendWS& w, const int32_t* group_start_dev,
               const int32_t* ids, const int32_t* pos, int n_tok, int n_groups, const int32_t* prefix_len,
               const int32_t* prefix_blocks, int max_blocks, const int32_t* extra_slot, const int32_t* n_extra,
               int max_extra, float temperature, const uint32_t* legal, int legal_words,
               const allie_outputs* out, void* kv_pool, int kv_pool_blocks, int32_t* status, hipStream_t st) {
  int rc;
  const int act = m->act_bf16;
  const int n1 = plan.n1, max_group = plan.max_group, max_rest = plan.max_rest, tile_q = plan.tile_q;
  const int64_t n_tiles = plan.n_tiles;
  const int32_t* group_start = group_start_dev ? group_start_dev : w.group_start;
  // the tree kernel shares a group's prefix across a tile of queries; groups of
  // one token (decode) stream it with one wave per query.  A batch that mixes
  // them (decode steps plus new games' prefixes) puts the one-token groups
  // first: those n1 tokens go to the wave kernel, the rest to the tree kernel.
  const bool tree = act && max_group > 1;
  // groups of at most 16 tokens (MCTS children of one node) take the fan
  // kernel instead: the waves of a (group, head) split the prefix
  const bool fan = tree && max_rest <= FAN_MAX_Q;
  if (tree && !fan) HIP_TRY(launch_extend_tiles(group_start, n1, n_groups, tile_q, w.tiles, st));
  ExtendPrepArgs pa{};
  pa.n = n_tok;
  pa.n_groups = n_groups;
  pa.max_blocks = max_blocks;
  pa.max_extra = max_extra;
  pa.pool_blocks = kv_pool_blocks;
  pa.n_positions = m->cfg.n_positions;
  pa.pos = pos;
  pa.group_start = group_start;
  pa.prefix_len = prefix_len;
  pa.prefix_blocks = prefix_blocks;
  pa.extra_slot = extra_slot;
  pa.n_extra = n_extra;
  pa.self_slot = w.self_slot;
  pa.status = status ? status : w.status;
  HIP_TRY(launch_extend_prepare(pa, st));

  EmbedArgs ea{};
  ea.ids = ids;
  ea.pos = pos;
  ea.T = n_tok;
  ea.d = m->d;
  ea.vocab = m->V;
  ea.n_positions = m->cfg.n_positions;
  ea.wte = m->wte;
  ea.wpe = m->wpe;
  ea.ctrl = m->ctrl;
  ea.ln_g = m->layers[0].ln1_g;
  ea.ln_b = m->layers[0].ln1_b;
  ea.eps = m->cfg.eps;
  ea.h = w.h;
  ea.x = w.x;
  ea.act_bf16 = act;
  HIP_TRY(launch_embed_ln(ea, st));

  ExtendAttnArgs xa{};
  xa.qkv = w.qkv;
  xa.pos = pos;
  xa.n = n_tok;
  xa.one_token_groups = n1 == n_groups;
  xa.n_head = m->H;
  xa.group_start = group_start;
  xa.n_groups = n_groups;
  xa.prefix_len = prefix_len;
  xa.prefix_blocks = prefix_blocks;
  xa.max_blocks = max_blocks;
  xa.extra_slot = extra_slot;
  xa.n_extra = n_extra;
  xa.max_extra = max_extra;
  xa.tiles = w.tiles;
  xa.n_tiles = (int)n_tiles;
  xa.tile_q = tile_q;
  xa.pool = kv_pool;
  xa.pool_blocks = kv_pool_blocks;
  xa.n_layer = m->L;
  xa.scale = 0.125f;  // 1 / sqrt(64)
  xa.out = w.attn;
  xa.act_bf16 = act;
  xa.self_slot = w.self_slot;  // written by the prepare step above
  xa.head_group = m->tree_heads;

  // one-token groups (decode steps) [0, n_dec) stream their keys with one
  // wave per (token, head), the games with the most keys first (bf16)
  const int n_dec = tree ? n1 : (xa.one_token_groups ? n_tok : 0);
  // too few (token, head) rows to fill the device with one wave each (an
  // MCTS leaf: 16): a workgroup of waves splits each row's keys
  const bool split_dec = act && n_dec > 0 && (int64_t)n_dec * m->H <= DECODE_SPLIT_MAX_ROWS;
  if (act && n_dec > 0 && !split_dec) HIP_TRY(launch_decode_order(xa, n_dec, w.order, st));
  auto launch_decode = [&](int nd) -> hipError_t {
    ExtendAttnArgs wa = xa;
    wa.n = nd == n_groups ? n_tok : nd;
    wa.one_token_groups = nd == n_groups ? xa.one_token_groups : 1;
    if (split_dec) return launch_attn_extend_split(wa, st);
    wa.order = (act && wa.one_token_groups) ? w.order : nullptr;
    return launch_attn_extend_wave(wa, st);
  };
  const Acts acts{w.h, w.x, w.qkv, w.attn, w.ff, w.part, w.wdq};
  const void* final_add = nullptr;
  const float* h_final = nullptr;
  rc = run_layers(m, acts, n_tok, w.self_slot, kv_pool, kv_pool_blocks, true,
                  [&](int layer) -> int {
                    xa.layer = layer;
                    if (tree) {
                      if (n1 > 0) {
                        HIP_TRY(probe_mark(ALLIE_PROBE_DECODE, true, st));
                        HIP_TRY(launch_decode(n1));
                        HIP_TRY(probe_mark(ALLIE_PROBE_DECODE, false, st));
                      }
                      HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, true, st));
                      if (fan)
                        HIP_TRY(launch_attn_extend_fan(xa, n1, n_groups, 0, st));
                      else
                        HIP_TRY(launch_attn_extend_tree(xa, st));
                      HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, false, st));
                    } else {
                      HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, true, st));
                      HIP_TRY(probe_mark(ALLIE_PROBE_DECODE, true, st));
                      HIP_TRY(launch_decode(n_groups));
                      HIP_TRY(probe_mark(ALLIE_PROBE_DECODE, false, st));
                      HIP_TRY(probe_mark(ALLIE_PROBE_ATTN, false, st));
                    }
                    return ALLIE_OK;
                  },
                  st, nullptr, &h_final, &final_add);
  if (rc) return rc;
  return run_heads(m, w.h, final_add, nullptr, n_tok, w.hx, w.z, temperature, legal, legal_words, out, w.part, st);
}

}  // namespace

extern "C" {

int allie_extend(allie_model* m, const int32_t* ids, const int32_t* pos, int n_tok,
                 const int32_t* group_start_host, int n_groups, const int32_t* prefix_len,
                 const int32_t* prefix_blocks, int max_blocks, const int32_t* extra_slot,
                 const int32_t* n_extra, int max_extra, float temperature, const uint32_t* legal,
                 int legal_words, const allie_outputs* out, void* kv_pool, int kv_pool_blocks,
                 int32_t* status, void* workspace, size_t workspace_bytes, void* stream) {
  ExtendPlan plan;
  int rc = extend_check(m, ids, pos, n_tok, group_start_host, n_groups, prefix_len, prefix_blocks, max_blocks,
                        extra_slot, n_extra, max_extra, legal, legal_words, out, kv_pool, kv_pool_blocks, &plan);
  if (rc) return rc;
  if (!workspace) return fail(ALLIE_ERR_ARG, "bad extend arguments");
  ExtendWS w = layout_extend(m, n_tok, n_groups, (char*)workspace, true);
  hipStream_t st = (hipStream_t)stream;
  // A large extend (MCTS tree levels; or a decode step of many games, whose
  // HBM-bound attention then runs beside the other half's latency-bound
  // projections) runs as two halves of consecutive groups on the model's two
  // streams, as a large prefill does: groups never share keys they write, and
  // each reads only its own prefix.
  if ((split_size(m, n_tok) || split_decode_size(m, plan.n1)) && n_groups >= 2 && m->fork) {
    int gc = 1;
    while (gc < n_groups - 1 && 2 * (int64_t)group_start_host[gc] < n_tok) ++gc;
    const int t0 = group_start_host[gc];
    std::vector<int32_t> gs1((size_t)(n_groups - gc) + 1);
    for (int g = gc; g <= n_groups; ++g) gs1[(size_t)(g - gc)] = group_start_host[g] - t0;
    ExtendPlan p0, p1;
    allie_outputs o1 = *out;
    auto shift = [&](auto* q, int64_t k) { return q ? q + k : q; };
    o1.logits = shift(out->logits, (int64_t)t0 * m->V);
    o1.logits_raw = shift(out->logits_raw, (int64_t)t0 * m->V);
    o1.value = out->value + t0;
    o1.time = out->time + t0;
    o1.top1 = out->top1 + t0;
    o1.max_logit = out->max_logit + t0;
    o1.lse = out->lse + t0;
    const uint32_t* legal1 = legal ? legal + (int64_t)t0 * legal_words : nullptr;
    const int32_t *ids1 = ids + t0, *pos1 = pos + t0, *pl1 = prefix_len + gc,
                  *pb1 = prefix_blocks ? prefix_blocks + (int64_t)gc * max_blocks : nullptr,
                  *es1 = extra_slot + (int64_t)t0 * max_extra, *ne1 = n_extra + t0;
    if (!extend_check(m, ids, pos, t0, group_start_host, gc, prefix_len, prefix_blocks, max_blocks, extra_slot,
                      n_extra, max_extra, legal, legal_words, out, kv_pool, kv_pool_blocks, &p0) &&
        !extend_check(m, ids1, pos1, n_tok - t0, gs1.data(), n_groups - gc, pl1, pb1, max_blocks, es1, ne1,
                      max_extra, legal1, legal_words, &o1, kv_pool, kv_pool_blocks, &p1)) {
      const ExtendWS w0 = layout_extend(m, t0, gc, (char*)workspace, true);
      const ExtendWS w1 = layout_extend(m, n_tok - t0, n_groups - gc, (char*)workspace + w0.total, true);
      int dev = -1;
      if (w0.total + w1.total <= workspace_bytes && hipGetDevice(&dev) == hipSuccess && dev == m->device) {
        HIP_TRY(hipEventRecord(m->fork, st));
        for (int i = 0; i < 2; ++i) HIP_TRY(hipStreamWaitEvent(m->side[i], m->fork, 0));
        if ((rc = upload_i32(m, w0.group_start, group_start_host, (size_t)gc + 1, m->side[0]))) return rc;
        if ((rc = extend_run(m, p0, w0, nullptr, ids, pos, t0, gc, prefix_len, prefix_blocks, max_blocks, extra_slot,
                             n_extra, max_extra, temperature, legal, legal_words, out, kv_pool, kv_pool_blocks,
                             nullptr, m->side[0])))
          return rc;
        if ((rc = upload_i32(m, w1.group_start, gs1.data(), gs1.size(), m->side[1]))) return rc;
        if ((rc = extend_run(m, p1, w1, nullptr, ids1, pos1, n_tok - t0, n_groups - gc, pl1, pb1, max_blocks, es1, ne1,
                             max_extra, temperature, legal1, legal_words, &o1, kv_pool, kv_pool_blocks, nullptr,
                             m->side[1])))
          return rc;
        for (int i = 0; i < 2; ++i) {
          HIP_TRY(hipEventRecord(m->join[i], m->side[i]));
          HIP_TRY(hipStreamWaitEvent(st, m->join[i], 0));
        }
        if (status) hipLaunchKernelGGL(or_status_kernel, dim3(1), dim3(64), 0, st, status, w0.status, w1.status);
        return ALLIE_OK;
      }
    }
  }
  if (workspace_bytes < w.total)
    return fail(ALLIE_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, w.total);
  if ((rc = upload_i32(m, w.group_start, group_start_host, (size_t)n_groups + 1, st))) return rc;
  return extend_run(m, plan, w, nullptr, ids, pos, n_tok, n_groups, prefix_len, prefix_blocks, max_blocks,
                    extra_slot, n_extra, max_extra, temperature, legal, legal_words, out, kv_pool, kv_pool_blocks,
                    status, st);
}

int allie_extend_noalloc(allie_model* m, const int32_t* ids, const int32_t* pos, int n_tok,
                         const int32_t* group_start_host, const int32_t* group_start, int n_groups,
                         const int32_t* prefix_len, const int32_t* prefix_blocks, int max_blocks,
                         const int32_t* extra_slot, const int32_t* n_extra, int max_extra, float temperature,
                         const uint32_t* legal, int legal_words, const allie_outputs* out, void* kv_pool,
                         int kv_pool_blocks, int32_t* status, void* stream) {
  ExtendPlan plan;
  int rc = extend_check(m, ids, pos, n_tok, group_start_host, n_groups, prefix_len, prefix_blocks, max_blocks,
                        extra_slot, n_extra, max_extra, legal, legal_words, out, kv_pool, kv_pool_blocks, &plan);
  if (rc) return rc;
  if (!group_start) return fail(ALLIE_ERR_ARG, "group_start (device copy) is required");
  if (n_tok > ALLIE_NOALLOC_MAX_TOKENS)
    return fail(ALLIE_ERR_WORKSPACE, "allie_extend_noalloc: %d tokens (max %d)", n_tok, ALLIE_NOALLOC_MAX_TOKENS);
  // no fp8 widening buffer: at these row counts no GEMM runs on the persistent kernel
  const size_t need = layout_extend(m, n_tok, n_groups, nullptr, false).total;
  if (need > (size_t)ALLIE_NOALLOC_SCRATCH_BYTES)
    return fail(ALLIE_ERR_WORKSPACE, "allie_extend_noalloc: %d tokens in %d groups need %zu bytes of scratch (max %zu)",
                n_tok, n_groups, need, (size_t)ALLIE_NOALLOC_SCRATCH_BYTES);
  char* base = (char*)scratch_ptr(m->device);
  if (!base) return fail(ALLIE_ERR_STATE, "scratch of device %d not initialised", m->device);
  ExtendWS w = layout_extend(m, n_tok, n_groups, base, false);
  return extend_run(m, plan, w, group_start, ids, pos, n_tok, n_groups, prefix_len, prefix_blocks, max_blocks,
                    extra_slot, n_extra, max_extra, temperature, legal, legal_words, out, kv_pool, kv_pool_blocks,
                    status, (hipStream_t)stream);
}

int allie_probe_begin(int kind, int max_launches) {
  if (kind < ALLIE_PROBE_QKV || kind > ALLIE_PROBE_DECODE || max_launches <= 0)
    return fail(ALLIE_ERR_ARG, "bad probe arguments");
  for (auto e : g_probe.start) (void)hipEventDestroy(e);
  for (auto e : g_probe.stop) (void)hipEventDestroy(e);
  g_probe = Probe();
  g_probe.start.resize(max_launches);
  g_probe.stop.resize(max_launches);
  for (int i = 0; i < max_launches; ++i) {
    HIP_TRY(hipEventCreate(&g_probe.start[i]));
    HIP_TRY(hipEventCreate(&g_probe.stop[i]));
  }
  g_probe.kind = kind;
  return ALLIE_OK;
}

int allie_probe_span(float* span_ms_host) {
  if (!span_ms_host) return fail(ALLIE_ERR_ARG, "NULL argument");
  const int n = g_probe.n;
  std::vector<std::pair<float, float>> iv((size_t)n);
  for (int i = 0; i < n; ++i) {
    HIP_TRY(hipEventSynchronize(g_probe.stop[i]));
    HIP_TRY(hipEventElapsedTime(&iv[i].first, g_probe.start[0], g_probe.start[i]));
    HIP_TRY(hipEventElapsedTime(&iv[i].second, g_probe.start[0], g_probe.stop[i]));
  }
  std::sort(iv.begin(), iv.end());
  float span = 0.f, lo = 0.f, hi = 0.f;
  for (int i = 0; i < n; ++i) {
    if (i == 0 || iv[i].first > hi) {
      span += hi - lo;
      lo = iv[i].first;
      hi = iv[i].second;
    } else if (iv[i].second > hi) {
      hi = iv[i].second;
    }
  }
  if (n > 0) span += hi - lo;
  *span_ms_host = span;
  return ALLIE_OK;
}

int allie_probe_end(float* total_ms_host, int* n_launches_host) {
  if (!total_ms_host || !n_launches_host) return fail(ALLIE_ERR_ARG, "NULL argument");
  float tot = 0.f;
  const int n = g_probe.n;
  for (int i = 0; i < n; ++i) {
    HIP_TRY(hipEventSynchronize(g_probe.stop[i]));
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, g_probe.start[i], g_probe.stop[i]));
    tot += ms;
  }
  for (auto e : g_probe.start) (void)hipEventDestroy(e);
  for (auto e : g_probe.stop) (void)hipEventDestroy(e);
  g_probe = Probe();
  *total_ms_host = tot;
  *n_launches_host = n;
  return ALLIE_OK;
}

int allie_gemm(const void* A, const void* W, const float* bias, const float* scale, void* C,
               float* R, int M, int N, int K, int epi, int wtype, int out_f32, void* wdq, void* stream) {
  if (!A || !W || M < 0 || N <= 0 || K <= 0) return fail(ALLIE_ERR_ARG, "bad gemm arguments");
  if (epi < EPI_STORE || epi > EPI_RESID || wtype < W_BF16 || wtype > W_FP8)
    return fail(ALLIE_ERR_ARG, "bad gemm mode");
  if ((epi == EPI_RESID && !R) || (epi != EPI_RESID && !C) || (wtype == W_FP8 && !scale))
    return fail(ALLIE_ERR_ARG, "missing gemm output/scale");
  GemmArgs g{};
  g.A = A;
  g.W = W;
  g.bias = bias;
  g.scale = scale;
  g.C = C;
  g.R = R;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldc = N;
  g.ldr = N;
  g.epi = epi;
  g.wtype = wtype;
  g.out_f32 = wtype == W_F32 ? 1 : out_f32;
  g.wdq = wtype == W_FP8 ? wdq : nullptr;
  if (wtype != W_F32 && !gemm_mfma_supported(g) && !gemm_skinny_supported(g))
    return fail(ALLIE_ERR_ARG,
                "gemm needs N %% 128 == 0 and K %% 32 == 0, or M <= %d, N %% 4 == 0 and K %% 8 == 0 (M=%d N=%d K=%d)",
                SKINNY_MAX_M, M, N, K);
  if (wtype == W_FP8 && out_f32) return fail(ALLIE_ERR_ARG, "fp8 gemm has bf16 output only");
  if (wtype != W_F32 && out_f32 && epi != EPI_STORE)
    return fail(ALLIE_ERR_ARG, "fp32 output only with the store epilogue");
  HIP_TRY(launch_gemm(g, (hipStream_t)stream));
  return ALLIE_OK;
}

int allie_gemm_splitk(const void* A, const void* W, const float* bias, const float* scale, void* C,
                      float* R, int M, int N, int K, int epi, int wtype, int out_f32, int split_k,
                      float* part, size_t part_bytes_, void* stream) {
  if (!A || !W || M <= 0 || N <= 0 || K <= 0 || !part) return fail(ALLIE_ERR_ARG, "bad gemm arguments");
  if (epi < EPI_STORE || epi > EPI_RESID || (wtype != W_BF16 && wtype != W_FP8))
    return fail(ALLIE_ERR_ARG, "bad split-K gemm mode");
  if ((epi == EPI_RESID && !R) || (epi != EPI_RESID && !C) || (wtype == W_FP8 && !scale))
    return fail(ALLIE_ERR_ARG, "missing gemm output/scale");
  if (out_f32 && (wtype == W_FP8 || epi != EPI_STORE))
    return fail(ALLIE_ERR_ARG, "fp32 output only with bf16 weights and the store epilogue");
  const int s = split_k > 0 ? split_k : gemm_split_factor(M, N, K);
  if (N % 128 != 0 || K % 32 != 0 || (K / 32) % s != 0)
    return fail(ALLIE_ERR_ARG, "split-K gemm needs N %% 128 == 0, K %% 32 == 0 and K / 32 divisible by %d", s);
  if (part_bytes_ < (size_t)s * M * N * 4)
    return fail(ALLIE_ERR_WORKSPACE, "partials need %zu bytes", (size_t)s * M * N * 4);
  GemmArgs g{};
  g.A = A;
  g.W = W;
  g.bias = bias;
  g.scale = scale;
  g.C = C;
  g.R = R;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldc = N;
  g.ldr = N;
  g.epi = epi;
  g.wtype = wtype;
  g.out_f32 = out_f32;
  g.split = s;
  g.part = part;
  HIP_TRY(launch_gemm(g, (hipStream_t)stream));
  return ALLIE_OK;
}

int allie_gemm_split_factor(int M, int N, int K) { return gemm_split_factor(M, N, K); }

int allie_attn_varlen(const void* qkv, const int32_t* cu_seqlens, const int32_t* tiles,
                      int n_tiles, int n_seq, int n_tokens, int n_head, int head_dim,
                      float scale, void* out, int act_bf16, int32_t* order_ws, void* stream) {
  if (!qkv || !cu_seqlens || !out || (act_bf16 && !order_ws) || head_dim != 64 || n_head <= 0)
    return fail(ALLIE_ERR_ARG, "bad attention arguments");
  AttnVarlenArgs a{};
  a.qkv = qkv;
  a.cu_seqlens = cu_seqlens;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.B = n_seq;
  a.T = n_tokens;
  a.n_head = n_head;
  a.head_dim = head_dim;
  a.scale = scale;
  a.out = out;
  a.act_bf16 = act_bf16;
  a.order = order_ws;
  HIP_TRY(launch_attn_varlen(a, (hipStream_t)stream));
  return ALLIE_OK;
}

int allie_layernorm(const float* h, const int32_t* row_idx, int rows, int rows_out, int d,
                    const float* g, const float* b, float eps, void* y, int act_bf16,
                    void* stream) {
  if (!h || !g || !b || !y || rows < 0 || rows_out < rows || d % 256 != 0 || d > 2048)
    return fail(ALLIE_ERR_ARG, "bad layernorm arguments");
  LNArgs a{};
  a.h = h;
  a.row_idx = row_idx;
  a.rows = rows;
  a.rows_out = rows_out;
  a.d = d;
  a.g = g;
  a.b = b;
  a.eps = eps;
  a.y = y;
  a.act_bf16 = act_bf16;
  HIP_TRY(launch_layernorm(a, (hipStream_t)stream));
  return ALLIE_OK;
}

}  // extern "C"
