// Attention of new tokens over a paged KV cache: MCTS tree expansion and
// continuous-batching decode.
//
// The reference has no KV cache: every MCTS leaf and every appended move is a
// full recompute of the game prefix at batch 1 (src/evaluation/decode.py:
// 356-360, README.md:80).  What such a recompute yields at the new token is
// softmax(q K^T / 8) V over all earlier tokens of the same game plus the token
// itself, which is what these kernels compute from cached keys and values:
//
//   keys of token i = its group's shared prefix (a root's game, or a decode
//                     slot's context), read through the group's block table,
//                     then the token's private keys (a search node's
//                     ancestors and the node itself), read slot by slot.
//
// Pool layout (one block = 16 positions of every layer; NB = pool blocks):
//   [layer][NB blocks][k|v][head][16][64]  (bf16, or fp32 in the fp32 check mode)
// so one (layer, block, k|v, head) is a contiguous 2 KiB (bf16) row group,
// and the keys one layer's kernel reads lie in that layer's 1 / L of the
// pool: random 2 KiB reads over 2 GiB run at 6.9 TB/s against 6.1 over
// 48 GiB (measured), so the per-layer window keeps the page walks local.
//
// attn_extend_wave_kernel  -- one wave per (token, head); lane l owns key
//   l / 4 of a 16-key block and head dims 16 (l % 4) .. +15.  Streams the keys
//   once per query, the next block's keys and values loading while one is
//   reduced: the decode kernel (groups of one token).
// attn_extend_tree_kernel  -- a workgroup per (64-query tile of a group,
//   head): the group's prefix keys are staged through LDS once per tile and
//   multiplied on the MFMA units (S^T = K Q^T, O^T = V^T P^T, as in the
//   varlen prefill kernel); each query's private keys follow in registers.
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int HD = 64;
constexpr int KT = 64;           // prefix keys per LDS tile (4 pool blocks)
constexpr int PREP_THREADS = 1024;

// element offset of (block, layer, k|v, head, offset-in-block, dim 0)
ALLIE_DEV int64_t pool_off(int64_t blk, int n_blocks, int layer, int kv, int H, int head, int off) {
  return (((((int64_t)layer * n_blocks + blk) * 2 + kv) * H + head) * KV_BLOCK + off) * (int64_t)HD;
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(PREP_THREADS) void extend_prepare_kernel(ExtendPrepArgs a) {
  int bad = 0;
  for (int i = threadIdx.x; i < a.n; i += PREP_THREADS) {
    const int ne = a.n_extra[i];
    int self = -1;
    if (ne < 1 || ne > a.max_extra) {
      bad |= 1;
    } else {
      for (int e = 0; e < ne; ++e) {
        const int sl = a.extra_slot[(int64_t)i * a.max_extra + e];
        if (sl < 0 || (sl >> 4) >= a.pool_blocks) bad |= 2;
      }
      self = a.extra_slot[(int64_t)i * a.max_extra + ne - 1];
    }
    a.self_slot[i] = self;
    const int p = a.pos[i];
    if (p < 0 || p >= a.n_positions) bad |= 4;
  }
  for (int g = threadIdx.x; g < a.n_groups; g += PREP_THREADS) {
    const int P = a.prefix_len[g];
    const int nb = (P + KV_BLOCK - 1) / KV_BLOCK;
    if (P < 0 || nb > a.max_blocks) {
      bad |= 2;
      continue;
    }
    for (int b = 0; b < nb; ++b) {
      const int blk = a.prefix_blocks[(int64_t)g * a.max_blocks + b];
      if (blk < 0 || blk >= a.pool_blocks) bad |= 2;
    }
  }
  const int b1 = __syncthreads_or(bad & 1), b2 = __syncthreads_or(bad & 2), b4 = __syncthreads_or(bad & 4);
  if (threadIdx.x == 0 && a.status) *a.status = (b1 ? 1 : 0) | (b2 ? 2 : 0) | (b4 ? 4 : 0);
}

// Tile list of the tree kernel: (g << 8) | t for t < ceil(size_g / tq), groups
// in order.  One workgroup; exclusive scan of the per-group tile counts.
__global__ __launch_bounds__(PREP_THREADS) void extend_tiles_kernel(const int32_t* __restrict__ group_start,
                                                                    int g0, int G, int tq, int32_t* __restrict__ tiles) {
  __shared__ int sh[PREP_THREADS / 64 + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int carry = 0;
  for (int base = g0; base < G; base += PREP_THREADS) {
    const int g = base + threadIdx.x;
    const int nt = g < G ? (group_start[g + 1] - group_start[g] + tq - 1) / tq : 0;
    int x = nt;  // inclusive wave scan
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) sh[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
      int s = 0;
      for (int w = 0; w < PREP_THREADS / 64; ++w) {
        const int v = sh[w];
        sh[w] = s;
        s += v;
      }
      sh[PREP_THREADS / 64] = s;
    }
    __syncthreads();
    const int first = carry + sh[wave] + x - nt;
    for (int t = 0; t < nt; ++t) tiles[first + t] = (g << 8) | t;
    carry += sh[PREP_THREADS / 64];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
template <typename T>
ALLIE_DEV void load16(const T* p, float (&v)[16]);
template <>
ALLIE_DEV void load16<bf16_t>(const bf16_t* p, float (&v)[16]) {
  const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[2 * j] = bf2f(w[j] & 0xffffu);
    v[2 * j + 1] = bf2f(w[j] >> 16);
  }
}
template <>
ALLIE_DEV void load16<float>(const float* p, float (&v)[16]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4 f = reinterpret_cast<const float4*>(p)[j];
    v[4 * j] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
}

// 16 elements of a key or value row as stored (bf16: 32 B, fp32: 64 B)
template <typename T>
struct Row16 {
  uint4 v[sizeof(T) * 16 / 16];
};
template <typename T>
ALLIE_DEV void fetch16(const T* p, Row16<T>& r) {
#pragma unroll
  for (int j = 0; j < (int)(sizeof(T)); ++j) r.v[j] = reinterpret_cast<const uint4*>(p)[j];
}
template <typename T>
ALLIE_DEV void widen16(const Row16<T>& r, float (&v)[16]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t w[4] = {r.v[j].x, r.v[j].y, r.v[j].z, r.v[j].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[8 * j + 2 * t] = bf2f(w[t] & 0xffffu);
        v[8 * j + 2 * t + 1] = bf2f(w[t] >> 16);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[4 * j] = __uint_as_float(r.v[j].x);
      v[4 * j + 1] = __uint_as_float(r.v[j].y);
      v[4 * j + 2] = __uint_as_float(r.v[j].z);
      v[4 * j + 3] = __uint_as_float(r.v[j].w);
    }
  }
}

// Order of the decode tokens (one-token groups 0 .. n - 1) for the wave
// kernel: most keys first, so the longest games do not start last.  One
// workgroup, a counting sort over 64 bins of 16 keys (order within a bin is
// arbitrary; every token's result is independent of it).
constexpr int ORDER_BINS = 64;
__global__ __launch_bounds__(PREP_THREADS) void decode_order_kernel(ExtendAttnArgs a, int n, int32_t* __restrict__ order) {
  __shared__ int bin[ORDER_BINS];
  if (threadIdx.x < ORDER_BINS) bin[threadIdx.x] = 0;
  __syncthreads();
  auto bin_of = [&](int i) {
    int E = a.n_extra[i];
    E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
    const int keys = max(min(a.prefix_len[i], a.pos[i]), 0) + E;
    return ORDER_BINS - 1 - min(keys / KV_BLOCK, ORDER_BINS - 1);  // bin 0: the most keys
  };
  for (int i = threadIdx.x; i < n; i += PREP_THREADS) atomicAdd(&bin[bin_of(i)], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int b = 0; b < ORDER_BINS; ++b) {
      const int c = bin[b];
      bin[b] = acc;
      acc += c;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += PREP_THREADS) order[atomicAdd(&bin[bin_of(i)], 1)] = i;
}

template <int CTRL>
ALLIE_DEV float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
ALLIE_DEV float readlane_f(float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); }

// bf16: held to 128 registers, four waves per SIMD (the fp32 check mode
// would spill there)
template <typename T>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 4 : 1) void attn_extend_wave_kernel(ExtendAttnArgs a) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int H = a.n_head, d = H * HD;
  if (wid >= (int64_t)a.n * H) return;  // no barriers below: whole waves leave
  const int i = a.order ? a.order[wid / H] : (int)(wid / H), head = (int)(wid % H);
  const int lane = threadIdx.x & 63;
  const int kj = lane >> 2, dq = (lane & 3) * 16;
  // group of token i: group_start[g] <= i < group_start[g + 1]
  int lo = i, hi = a.n_groups;
  if (!a.one_token_groups) {
    lo = 0;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.group_start[mid] <= i) lo = mid; else hi = mid;
    }
  }
  const int g = lo;
  const T* __restrict__ qkv = reinterpret_cast<const T*>(a.qkv);
  const T* __restrict__ pool = reinterpret_cast<const T*>(a.pool);
  const float sl2 = a.scale * 1.4426950408889634f;  // scale * log2(e)
  // q: bf16 pairs as stored (dot products by v_dot2_f32_bf16, the scale
  // applied to the sum), or fp32 pre-scaled
  Row16<T> qr;
  fetch16<T>(qkv + (int64_t)i * 3 * d + head * HD + dq, qr);
  float q[16];
  if constexpr (sizeof(T) == 4) {
    widen16<T>(qr, q);
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] *= sl2;
  }

  // keys in chunks of 16 (lane's key kj of the chunk): first the visible
  // prefix, one pool block per chunk -- positions below both the group's
  // prefix length and the token's own position -- then the token's extras
  const int P = min(a.prefix_len[g], a.pos[i]);
  int nbp = (P + KV_BLOCK - 1) / KV_BLOCK;
  nbp = nbp < a.max_blocks ? nbp : a.max_blocks;
  int E = a.n_extra[i];
  E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
  const int nch = nbp + (E + KV_BLOCK - 1) / KV_BLOCK;
  const int32_t* btab = a.prefix_blocks + (int64_t)g * a.max_blocks;
  const int my_blk = lane < nbp ? btab[lane] : -1;  // the first 64 blocks of the row
  // key kj of chunk c: offset of its key row, visible or not.  A key that is
  // not visible still reads a written row, one whose product with p = 0 is
  // zero (unwritten pool memory may hold NaN patterns): past the prefix the
  // block's first position, past the private keys the token's own slot
  // (written by this layer's QKV projection).  A block outside the pool
  // (a batch the prepare step flags) reads block 0.
  auto locate = [&](int c, int64_t& off, bool& ok) {
    int blk, kpos;
    if (c < nbp) {
      blk = c < 64 ? __builtin_amdgcn_readlane(my_blk, c) : btab[c];
      ok = c * KV_BLOCK + kj < P;
      kpos = ok ? kj : 0;
    } else {
      const int e = (c - nbp) * KV_BLOCK + kj;
      const int sl = a.extra_slot[(int64_t)i * a.max_extra + min(e, E - 1)];
      blk = sl >> 4;
      kpos = sl & 15;
      ok = e < E && sl >= 0;
    }
    const bool in_pool = blk >= 0 && blk < a.pool_blocks;
    ok = ok && in_pool;
    off = pool_off(in_pool ? blk : 0, a.pool_blocks, a.layer, 0, H, head, in_pool ? kpos : 0) + dq;
  };

  float m_run = -INFINITY, l_run = 0.f, acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  const int64_t voff = (int64_t)H * KV_BLOCK * HD;  // k -> v of the same (block, layer, head)
  // one chunk's keys and values (kr, vr) into the running softmax
  auto reduce_chunk = [&](const Row16<T>& kr, const Row16<T>& vr, bool ok) {
    float s = 0.f;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t qw[4] = {qr.v[j].x, qr.v[j].y, qr.v[j].z, qr.v[j].w};
        const uint32_t kw[4] = {kr.v[j].x, kr.v[j].y, kr.v[j].z, kr.v[j].w};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw[t]), __builtin_bit_cast(bf16x2_t, kw[t]),
                                              s, false);
      }
      s *= sl2;
    } else {
      float kv[16];
      widen16<T>(kr, kv);
#pragma unroll
      for (int j = 0; j < 16; ++j) s = fmaf(q[j], kv[j], s);
    }
    // cross-lane steps by DPP and lane reads, no LDS round trips: the 4 lanes
    // of a key (which share ok) sum their dims, then the max over the row's 4
    // keys and the 4 rows' maxima
    s += dpp_f<0xb1>(s);  // quad_perm [1, 0, 3, 2]
    s += dpp_f<0x4e>(s);  // quad_perm [2, 3, 0, 1]
    s = ok ? s : -INFINITY;
    float mb = fmaxf(s, dpp_f<0x124>(s));  // row_ror 4
    mb = fmaxf(mb, dpp_f<0x128>(mb));       // row_ror 8
    mb = fmaxf(fmaxf(readlane_f(mb, 0), readlane_f(mb, 16)), fmaxf(readlane_f(mb, 32), readlane_f(mb, 48)));
    const float m_new = fmaxf(m_run, mb);
    if (m_new == -INFINITY) return;  // nothing visible yet (wave-uniform)
    const float alpha = exp2f(m_run - m_new);
    const float p = ok ? exp2f(s - m_new) : 0.f;
    l_run = l_run * alpha + ((lane & 3) == 0 ? p : 0.f);
    // bf16: P enters the product with V rounded to bf16, the row sum takes
    // it unrounded (torch's bf16 SDPA)
    const float pv = sizeof(T) == 2 ? round_bf16(p) : p;
    float vv[16];
    widen16<T>(vr, vv);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = acc[j] * alpha + pv * vv[j];
    m_run = m_new;
  };
  auto fetch_chunk = [&](int c, Row16<T>& kr, Row16<T>& vr, bool& ok) {
    int64_t off;
    locate(c, off, ok);
    fetch16<T>(pool + off, kr);
    fetch16<T>(pool + off + voff, vr);
  };
  // private keys that fit one chunk (a decode step's own key) are requested
  // first, with no dependent round trip after the prefix's last chunk, and
  // reduced last
  const bool x1 = E > 0 && E <= KV_BLOCK;
  Row16<T> kX, vX;
  bool okX = false;
  if (x1) fetch_chunk(nbp, kX, vX, okX);
  const int nloop = x1 ? nbp : nch;
  // two register buffers: chunk c + 1 loads while chunk c is reduced
  Row16<T> kA, vA, kB, vB;
  bool okA = false, okB = false;
  if (nloop > 0) fetch_chunk(0, kA, vA, okA);
  for (int c = 0; c < nloop; c += 2) {
    if (c + 1 < nloop) fetch_chunk(c + 1, kB, vB, okB);
    reduce_chunk(kA, vA, okA);
    if (c + 1 >= nloop) break;
    if (c + 2 < nloop) fetch_chunk(c + 2, kA, vA, okA);
    reduce_chunk(kB, vB, okB);
  }
  if (x1) reduce_chunk(kX, vX, okX);
  // combine the 16 key lanes of each head-dim group
#pragma unroll
  for (int o = 4; o < 64; o <<= 1) {
    l_run += __shfl_xor(l_run, o, 64);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] += __shfl_xor(acc[j], o, 64);
  }
  l_run += __shfl_xor(l_run, 1, 64);
  l_run += __shfl_xor(l_run, 2, 64);
  if (kj != 0) return;
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  if constexpr (sizeof(T) == 2) {
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = pack_bf16x2(acc[2 * j] * inv, acc[2 * j + 1] * inv);
    uint4* o = reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(a.out) + (int64_t)i * d + head * HD + dq);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
  } else {
    float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + (int64_t)i * d + head * HD + dq);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = make_float4(acc[4 * j] * inv, acc[4 * j + 1] * inv, acc[4 * j + 2] * inv, acc[4 * j + 3] * inv);
  }
}

// Split decode kernel (bf16, one-token groups: token i is group i): one
// workgroup of NWV waves per (token, head), for batches with too few
// (token, head) rows to fill the device with one wave each.  An MCTS leaf
// has 16 rows: one wave per row walks its 5-8 key chunks one after another,
// each a dependent round trip to memory, while here wave w takes chunks
// w, w + NWV, ... so every chunk is requested at once.  Keys, visibility and
// rounding points are the wave kernel's (lane l holds key l / 4 of a chunk
// and head dims 16 (l % 4) .. +15; P rounded to bf16 for the product with V,
// the row sum unrounded); each wave keeps its own running max, and the waves'
// (max, sum, 64 accumulators) are combined through LDS.
template <int NWV>
__global__ __launch_bounds__(NWV * 64) void attn_extend_split_kernel(ExtendAttnArgs a) {
  const int H = a.n_head, d = H * HD;
  const int i = blockIdx.x / H, head = blockIdx.x - (blockIdx.x / H) * H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kj = lane >> 2, dq = (lane & 3) * 16;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);
  const bf16_t* __restrict__ pool = reinterpret_cast<const bf16_t*>(a.pool);
  const float sl2 = a.scale * 1.4426950408889634f;  // scale * log2(e)
  Row16<bf16_t> qr;
  fetch16<bf16_t>(qkv + (int64_t)i * 3 * d + head * HD + dq, qr);
  const int P = min(a.prefix_len[i], a.pos[i]);
  int nbp = (P + KV_BLOCK - 1) / KV_BLOCK;
  nbp = nbp < a.max_blocks ? nbp : a.max_blocks;
  int E = a.n_extra[i];
  E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
  const int nch = nbp + (E + KV_BLOCK - 1) / KV_BLOCK;
  const int32_t* btab = a.prefix_blocks + (int64_t)i * a.max_blocks;
  // as in the wave kernel: a key that is not visible reads a written row
  // (the block's first position, or the token's own slot) and gets p = 0
  auto locate = [&](int c, int64_t& off, bool& ok) {
    int blk, kpos;
    if (c < nbp) {
      blk = btab[c];
      ok = c * KV_BLOCK + kj < P;
      kpos = ok ? kj : 0;
    } else {
      const int e = (c - nbp) * KV_BLOCK + kj;
      const int sl = a.extra_slot[(int64_t)i * a.max_extra + min(e, E - 1)];
      blk = sl >> 4;
      kpos = sl & 15;
      ok = e < E && sl >= 0;
    }
    const bool in_pool = blk >= 0 && blk < a.pool_blocks;
    ok = ok && in_pool;
    off = pool_off(in_pool ? blk : 0, a.pool_blocks, a.layer, 0, H, head, in_pool ? kpos : 0) + dq;
  };
  float m_run = -INFINITY, l_run = 0.f, acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  const int64_t voff = (int64_t)H * KV_BLOCK * HD;
  auto reduce_chunk = [&](const Row16<bf16_t>& kr, const Row16<bf16_t>& vr, bool ok) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t qw[4] = {qr.v[j].x, qr.v[j].y, qr.v[j].z, qr.v[j].w};
      const uint32_t kw[4] = {kr.v[j].x, kr.v[j].y, kr.v[j].z, kr.v[j].w};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw[t]), __builtin_bit_cast(bf16x2_t, kw[t]), s,
                                            false);
    }
    s *= sl2;
    s += dpp_f<0xb1>(s);  // the 4 lanes of a key sum their dims
    s += dpp_f<0x4e>(s);
    s = ok ? s : -INFINITY;
    float mb = fmaxf(s, dpp_f<0x124>(s));  // max over the row's 4 keys, then the 4 rows
    mb = fmaxf(mb, dpp_f<0x128>(mb));
    mb = fmaxf(fmaxf(readlane_f(mb, 0), readlane_f(mb, 16)), fmaxf(readlane_f(mb, 32), readlane_f(mb, 48)));
    const float m_new = fmaxf(m_run, mb);
    if (m_new == -INFINITY) return;  // nothing visible yet (wave-uniform)
    const float alpha = exp2f(m_run - m_new);
    const float p = ok ? exp2f(s - m_new) : 0.f;
    l_run = l_run * alpha + ((lane & 3) == 0 ? p : 0.f);
    const float pv = round_bf16(p);
    float vv[16];
    widen16<bf16_t>(vr, vv);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = acc[j] * alpha + pv * vv[j];
    m_run = m_new;
  };
  auto fetch_chunk = [&](int c, Row16<bf16_t>& kr, Row16<bf16_t>& vr, bool& ok) {
    int64_t off;
    locate(c, off, ok);
    fetch16<bf16_t>(pool + off, kr);
    fetch16<bf16_t>(pool + off + voff, vr);
  };
  // two register buffers: this wave's next chunk loads while one is reduced
  Row16<bf16_t> kA, vA, kB, vB;
  bool okA = false, okB = false;
  if (wave < nch) fetch_chunk(wave, kA, vA, okA);
  for (int c = wave; c < nch; c += 2 * NWV) {
    if (c + NWV < nch) fetch_chunk(c + NWV, kB, vB, okB);
    reduce_chunk(kA, vA, okA);
    if (c + NWV >= nch) break;
    if (c + 2 * NWV < nch) fetch_chunk(c + 2 * NWV, kA, vA, okA);
    reduce_chunk(kB, vB, okB);
  }
  // the wave's 16 key lanes of each head-dim group, then its 4 groups' sums
#pragma unroll
  for (int o = 4; o < 64; o <<= 1) {
    l_run += __shfl_xor(l_run, o, 64);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] += __shfl_xor(acc[j], o, 64);
  }
  l_run += __shfl_xor(l_run, 1, 64);
  l_run += __shfl_xor(l_run, 2, 64);
  __shared__ float s_m[NWV], s_l[NWV], s_acc[NWV][HD];
  if (lane == 0) {
    s_m[wave] = m_run;
    s_l[wave] = l_run;
  }
  if (kj == 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) s_acc[wave][dq + j] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < NWV; ++w) mx = fmaxf(mx, s_m[w]);
  float l_tot = 0.f, o = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    const float f = s_m[w] == -INFINITY ? 0.f : exp2f(s_m[w] - mx);  // a wave that saw no visible key adds 0
    l_tot += s_l[w] * f;
    o += s_acc[w][lane] * f;
  }
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  reinterpret_cast<bf16_t*>(a.out)[(int64_t)i * d + head * HD + lane] = (bf16_t)f2bf(o * inv);
}

// ---------------------------------------------------------------------------
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// Tree kernel: a tile of TQ = 16 NW queries of one group (NW waves of 16
// queries on 16x16x32 MFMAs) and one head.  Keys arrive in chunks of 64,
// staged in LDS (K rows swizzled by kswz; V rows with 8-byte chunk j of row
// r at j ^ (4 ((r >> 1) & 1)), read transposed), DEPTH chunks loading into
// registers while one is multiplied.  P enters the PV product rounded to
// bf16 and the row sum unrounded, as in torch's bf16 SDPA.  First the
// group's prefix (query i sees positions below min(P, pos[i])), then the
// tile's private keys other than the tokens' own as columns: for each extra
// index e, a run of consecutive tokens whose e-th private key is the same
// pool slot (siblings' common ancestors) is one column, visible to exactly
// that run of queries.  Every (token, e) entry lands in exactly one column,
// so each query sees each of those keys once, whatever the slots are.  A
// token's own key and value (its last private key) are read by the token's
// own lanes from its slot and open its softmax.
constexpr int TREE_EB = 8;  // extra indices per column batch
// K rows (bf16, 128 B): 16-byte chunk c of row r at c ^ kswz(r)
ALLIE_DEV int kswz(int r) { return (r >> 1) & 7; }

// MH: the workgroup takes heads h0 .. h0 + hg - 1 (hg = a.head_group) of its
// tile in turn, with the positions, own slots, block table and columns
// loaded and built once, and its chunk sequence running on from one head
// into the next, so the next head's first chunks load while the current
// head's last are multiplied.  Each head's arithmetic is the one-head
// kernel's, in the same order (the same bits).  Needs a single column batch
// (max_extra <= TREE_EB).
template <int NW, int DEPTH, bool MH>
__global__ __launch_bounds__(NW * 64, 4) void attn_extend_tree_kernel(ExtendAttnArgs a) {
  constexpr int TQ = NW * 16, NT = NW * 64, PER = 512 / NT;  // PER: 16-byte K (and V) pieces per thread per chunk
  static_assert(NT >= TREE_MAX_BLOCKS, "one thread per staged block id");
  constexpr int NH = TQ / 64;                               // 64-token halves (column builder waves)
  constexpr int MAXC = TQ * TREE_EB;
  constexpr int NBUF = MH ? 2 : 1;  // LDS chunk buffers (MH: one staged while the other is multiplied)
  __shared__ __attribute__((aligned(1024))) uint16_t sK[NBUF * KT * HD];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[NBUF * KT * HD];
  __shared__ int32_t c_slot[MAXC + 64];   // column -> pool slot (-1: padding)
  __shared__ __attribute__((aligned(16))) uint32_t c_rng[MAXC + 64];  // column -> tile-local queries [lo, hi): lo | hi << 16
  __shared__ int32_t s_blk[TREE_MAX_BLOCKS];  // the prefix's pool blocks (-1: skipped)
  __shared__ int32_t s_tot[NH];

  const int hg = MH ? a.head_group : 1;
  const int h0 = blockIdx.y * hg;
  const int tile = a.tiles[blockIdx.x];
  const int g = tile >> 8, qt = tile & 255;
  const int H = a.n_head, d = H * HD, ld = 3 * d;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 15, lg = lane >> 4;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);
  const bf16_t* __restrict__ pool = reinterpret_cast<const bf16_t*>(a.pool);
  const int64_t voff = (int64_t)H * KV_BLOCK * HD;  // k -> v of the same (block, layer, head)
  // pool base of head h0 + hh at this layer
  const bf16_t* lbase0 = pool + ((int64_t)a.layer * a.pool_blocks * 2 * H + h0) * (KV_BLOCK * HD);
  auto hbase = [&](int hh) { return lbase0 + (int64_t)hh * (KV_BLOCK * HD); };
  const int64_t bstride = (int64_t)2 * H * KV_BLOCK * HD;
  const int q_first = a.group_start[g] + qt * TQ;
  const int ntok = min(TQ, a.group_start[g + 1] - q_first);
  const int P = max(a.prefix_len[g], 0);
  const int32_t* btab = a.prefix_blocks + (int64_t)g * a.max_blocks;
  const int nbp = min((P + KV_BLOCK - 1) / KV_BLOCK, a.max_blocks);  // blocks the prefix reads
  auto valid_blk = [&](int v) { return (v >= 0 && v < a.pool_blocks) ? v : -1; };
  // (from LDS only: a global load in the chunk loop, even one under a
  // condition never met, would make the wait before each staging cover the
  // chunks in flight)
  auto pblk = [&](int bi) { return bi < nbp ? s_blk[bi] : -1; };

  // ---- loads: block table, queries, positions, own slots ----------------
  // (issued together, none under a condition: a load under one gets a wait
  // of its own before the next is issued)
  // (the table row is read before the prefix length is known; no table: a
  // harmless read)
  const int bt_v = *(a.max_blocks > 0 ? btab + min(tid, a.max_blocks - 1) : a.group_start + g);
  const int qloc = wave * 16 + lq;  // tile-local query of this lane
  const bool q_ok = qloc < ntok;
  const int qi = q_first + (q_ok ? qloc : 0);
  const int pos_qi = a.pos[qi];
  const int self_v = a.self_slot[qi];
  bf16x8_t qf[2];  // B operand of S^T = K Q^T: query lq, dims 32 ks + 8 lg .. +7
  auto load_q = [&](int head) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(qkv + (int64_t)qi * ld + head * HD + 32 * ks + 8 * lg));
  };
  load_q(h0);
  if (tid < TREE_MAX_BLOCKS) s_blk[tid] = (tid < nbp && tid < a.max_blocks) ? valid_blk(bt_v) : -1;
  const int lim = q_ok ? min(P, pos_qi) : 0;

  // columns of extra indices [eb, eb + TREE_EB): wave h < NH builds tokens
  // 64 h .. 64 h + 63 (lane = token); a run never crosses two halves.  Ends
  // with the columns, their count in the return value and padding to 64.
  auto build_columns = [&](int eb) -> int {
    int sl[TREE_EB];
    uint64_t M[TREE_EB], brk[TREE_EB];
    int tot = 0;
    const int t = wave * 64 + lane;
    if (wave < NH) {
      const int i = q_first + t;
      const bool tv = t < ntok;
      int E = tv ? a.n_extra[i] : 0;
      E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
#pragma unroll
      for (int e = 0; e < TREE_EB; ++e) {
        const int ee = eb + e;
        // the last private key is the token's own: its lanes read it from the
        // pool at self_slot (below), never from qkv, whose K/V columns an
        // extend leaves unwritten
        const int v = (ee < E - 1) ? a.extra_slot[(int64_t)i * a.max_extra + ee] : -1;
        sl[e] = (v >= 0 && (v >> 4) < a.pool_blocks) ? v : -1;
      }
#pragma unroll
      for (int e = 0; e < TREE_EB; ++e) {
        const int prev = __shfl_up(sl[e], 1, 64);
        const bool start = sl[e] >= 0 && (lane == 0 || prev != sl[e]);
        M[e] = __ballot(start);
        brk[e] = M[e] | ~__ballot(sl[e] >= 0);
        tot += __popcll(M[e]);
      }
      if (lane == 0) s_tot[wave] = tot;
    }
    __syncthreads();
    int ncols = 0;
#pragma unroll
    for (int h = 0; h < NH; ++h) ncols += s_tot[h];
    if (wave < NH) {
      int base = 0;
      for (int h = 0; h < wave; ++h) base += s_tot[h];
#pragma unroll
      for (int e = 0; e < TREE_EB; ++e) {
        if ((M[e] >> lane) & 1) {
          const int idx = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(M[e] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)M[e], 0));
          const uint64_t rest = lane < 63 ? brk[e] >> (lane + 1) : 0;
          const int hi = rest ? lane + 1 + __builtin_ctzll(rest) : 64;
          c_slot[idx] = sl[e];
          c_rng[idx] = (uint32_t)t | ((uint32_t)(wave * 64 + hi) << 16);
        }
        base += __popcll(M[e]);
      }
    }
    if (wave == NW - 1) {  // padding of the last chunk: never visible
      const int pad = ncols + lane;
      if (pad < ((ncols + 63) & ~63)) {
        c_slot[pad] = -1;
        c_rng[pad] = 0;
      }
    }
    __syncthreads();
    return ncols;
  };

  const float c2 = a.scale * 1.4426950408889634f;
  float m_run, l_run;
  f32x4_t o[4];  // O^T: dims 16 db + 4 lg .. +3 of query lq
  // A head's softmax opens with the token's own key and value (its last
  // private key), read from its slot by its own lanes; the columns carry only
  // the other private keys (a tree level's own keys would otherwise be one
  // column per query).  (self_slot: the prepare step's copy, one dependent
  // load instead of two.)  Needs the head's queries in qf.
  const int self_sl = (q_ok && self_v >= 0 && (self_v >> 4) < a.pool_blocks) ? self_v : -1;
  auto open_head = [&](int hh) {
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x4_t{};
    const bool has_self = self_sl >= 0;
    const bf16_t* row = hbase(hh) + (int64_t)(has_self ? self_sl >> 4 : 0) * bstride + (self_sl & 15) * HD;
    float sdot = 0.f;
    uint2 vs[4] = {};
    if (has_self) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(row + 32 * ks + 8 * lg);
        const u32x4_t qw = __builtin_bit_cast(u32x4_t, qf[ks]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sdot = fmaf(bf2f(qw[e] & 0xffffu), bf2f(kw[e] & 0xffffu), sdot);
          sdot = fmaf(bf2f(qw[e] >> 16), bf2f(kw[e] >> 16), sdot);
        }
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) vs[db] = *reinterpret_cast<const uint2*>(row + voff + 16 * db + 4 * lg);
    }
    sdot = xor32_sum(xor16_sum(sdot));  // the query's four lane groups hold 16 dims each
    if (has_self) {
      m_run = sdot;
      l_run = lg == 0 ? 1.f : 0.f;  // the row sum is split over the lane groups
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = f32x4_t{bf2f(vs[db].x & 0xffffu), bf2f(vs[db].x >> 16), bf2f(vs[db].y & 0xffffu), bf2f(vs[db].y >> 16)};
    }
  };
  // normalise and store head h0 + hh's output rows (no barriers)
  auto close_head = [&](int hh) {
    if (!q_ok) return;
    const float l_tot = xor32_sum(xor16_sum(l_run));
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    bf16_t* out = reinterpret_cast<bf16_t*>(a.out) + (int64_t)qi * d + (h0 + hh) * HD + 4 * lg;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      uint2 w;
      w.x = pack_bf16x2(o[db][0] * inv, o[db][1] * inv);
      w.y = pack_bf16x2(o[db][2] * inv, o[db][3] * inv);
      *reinterpret_cast<uint2*>(out + 16 * db) = w;
    }
  };
  open_head(0);
  const bool wave_busy = wave * 16 < ntok;  // a wave past the tile's tokens only stages keys
  const int trow = lq >> 2, tchunk = lq & 3;  // transposing read: key row within 4, 4-dim chunk
  const int nchp = (P + KT - 1) / KT;

  // chunk j (prefix chunks first, then columns from c_slot) of the head whose
  // pool base is hb into registers: this thread's piece it is key row
  // (tid + NT it) / 8, 16-byte chunk % 8; a key outside a kept block reads
  // block 0 and is zeroed at staging
  auto fetch = [&](const bf16_t* hb, int j, int ncp, uint4 (&kv)[PER], uint4 (&vv)[PER], bool (&okf)[PER]) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int cidx = tid + NT * it;
      const int key = cidx >> 3, c = cidx & 7;
      int blk, off;
      if (j < ncp) {
        const int p = j * KT + key;
        blk = p < P ? pblk(p >> 4) : -1;
        off = p & 15;
      } else {
        const int sl = c_slot[(j - ncp) * 64 + key];
        blk = sl >= 0 ? sl >> 4 : -1;
        off = sl & 15;
      }
      okf[it] = blk >= 0;
      const bf16_t* src = hb + (int64_t)max(blk, 0) * bstride + off * HD + c * 8;
      kv[it] = *reinterpret_cast<const uint4*>(src);
      vv[it] = *reinterpret_cast<const uint4*>(src + voff);
    }
  };
  auto stage = [&](const uint4 (&kv)[PER], const uint4 (&vv)[PER], const bool (&okf)[PER], int buf = 0) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int cidx = tid + NT * it;
      const int key = cidx >> 3, c = cidx & 7;
      const uint4 k4 = okf[it] ? kv[it] : make_uint4(0, 0, 0, 0);
      const uint4 v4 = okf[it] ? vv[it] : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(sK + buf * KT * HD + key * HD + ((c ^ kswz(key)) << 3)) = k4;
      *reinterpret_cast<uint4*>(sV + buf * KT * HD + key * HD + ((c ^ (((key >> 1) & 1) << 1)) << 3)) = v4;
    }
  };
  // LDS read addresses, fixed for every chunk: K row 16 kb + lq, 16-byte
  // chunk 4 ks + lg, whose swizzle (lq >> 1) & 7 does not depend on kb; V
  // rows 32 s2 + 16 h + 4 lg + trow read transposed at 4-dim chunk
  // 4 (db ^ vb) + tchunk, vb = (trow >> 1) & 1 (the row swizzle bit)
  const int ksw = (lq >> 1) & 7, vb = (trow >> 1) & 1;
  const uint16_t* kp0 = sK + lq * HD + ((lg ^ ksw) << 3);
  const uint16_t* kp1 = sK + lq * HD + (((4 + lg) ^ ksw) << 3);
  const uint16_t* vp = sV + (4 * lg + trow) * HD + 4 * tchunk;
  const uint16_t* vp0 = vp + 16 * vb;        // db even
  const uint16_t* vp1 = vp + 16 * (1 - vb);  // db odd
  // the lowest limit over the wave's queries: a prefix chunk of kept blocks
  // wholly below it needs no mask
  int lim_w = lim;
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) lim_w = min(lim_w, __shfl_xor(lim_w, sh, 64));
  lim_w = __builtin_amdgcn_readfirstlane(lim_w);
  auto compute = [&](int j, int ncp, int buf = 0) {
    // S^T = K Q^T: st[kb][r] is key 16 kb + 4 lg + r of query lq
    f32x4_t st[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      st[kb] = f32x4_t{};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t kf =
            __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>((ks ? kp1 : kp0) + buf * KT * HD + kb * 16 * HD));
        st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], st[kb], 0, 0, 0);
      }
    }
    if (j < ncp) {  // prefix: positions below the query's limit in a kept block
      const int k0 = j * KT;
      bool bok[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) bok[kb] = pblk((k0 >> 4) + kb) >= 0;
      if (!(k0 + KT <= lim_w && bok[0] && bok[1] && bok[2] && bok[3])) {  // uniform
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (!bok[kb] || k0 + 16 * kb + 4 * lg + r >= lim) st[kb][r] = -INFINITY;
      }
    } else {  // columns: visible to their run of queries
      const int cb = (j - ncp) * 64;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint4 rg = *reinterpret_cast<const uint4*>(c_rng + cb + 16 * kb + 4 * lg);
        const uint32_t rr[4] = {rg.x, rg.y, rg.z, rg.w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (qloc < (int)(rr[r] & 0xffffu) || qloc >= (int)(rr[r] >> 16)) st[kb][r] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[kb][r]);
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    u32x4_t pf[2];  // P^T of k-step s: keys 32 s + 4 lg + {0..3}, then 32 s + 16 + 4 lg + {0..3}
    if (m_new != -INFINITY) {  // uniform per query
      const float m_old = m_run;
      m_run = m_new;
      const float mc = m_new * c2;
      float p[4][4];
      float ls = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kb][r] = __builtin_amdgcn_exp2f(fmaf(st[kb][r], c2, -mc));
          ls += p[kb][r];
        }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        pf[s2] = u32x4_t{pack_bf16x2(p[2 * s2][0], p[2 * s2][1]), pack_bf16x2(p[2 * s2][2], p[2 * s2][3]),
                         pack_bf16x2(p[2 * s2 + 1][0], p[2 * s2 + 1][1]), pack_bf16x2(p[2 * s2 + 1][2], p[2 * s2 + 1][3])};
      // a query whose maximum did not move has alpha = exp2(0) = 1 exactly:
      // when no query of the wave moved, the rescale is skipped (same bits)
      if (__builtin_amdgcn_ballot_w64(m_new != m_old)) {
        const float alpha = __builtin_amdgcn_exp2f((m_old - m_new) * c2);
        l_run = l_run * alpha + ls;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] *= alpha;
      } else {
        l_run = l_run + ls;
      }
    } else {
      pf[0] = pf[1] = u32x4_t{0, 0, 0, 0};
    }
    // O^T += V^T P^T: A = V^T rows (dims 16 db + lq), k-slots as P^T's;
    // lane group lg reads keys 32 s + 4 lg + trow (and + 16) transposed
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t* vr = (db & 1 ? vp1 : vp0) + buf * KT * HD + 32 * s2 * HD + 16 * (db & 2);
        const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)vr));
        const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)(vr + 16 * HD)));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, u32x4_t{l2.x, l2.y, h2.x, h2.y}),
                                                        __builtin_bit_cast(bf16x8_t, pf[s2]), o[db], 0, 0, 0);
      }
  };

  // two chunks in flight: chunk j + 2 loads into the registers chunk j was
  // staged from while j is multiplied.  Every fetch in the loop is
  // unconditional (past the last chunk it re-reads the last, never staged):
  // a load under a condition makes the compiler's wait before the next
  // multiply cover the chunk just requested
  uint4 kA[PER] = {}, vA[PER] = {}, kB[PER] = {}, vB[PER] = {};
  bool oA[PER] = {}, oB[PER] = {};
  __syncthreads();  // s_blk is in
  if (nchp > 0) fetch(hbase(0), 0, nchp, kA, vA, oA);  // the prefix's first chunks load while the columns are built
  if (DEPTH > 1 && nchp > 1) fetch(hbase(0), 1, nchp, kB, vB, oB);
  if constexpr (MH) {
    // one column batch; the flat chunk sequence J runs over the heads: head
    // J / nch, its chunk J % nch
    const int ncols = build_columns(0);
    const int nch = nchp + (ncols + 63) / 64;
    const int NJ = nch * hg;
    // (only for 0 <= J < NJ, so nch > 0 and the head is one of the group's)
    auto fetchJ = [&](int J, uint4 (&kv)[PER], uint4 (&vv)[PER], bool (&okf)[PER]) {
      const int hh = J / nch;
      fetch(hbase(hh), J - hh * nch, nchp, kv, vv, okf);
    };
    if (nchp < 1 && NJ > 0) fetchJ(0, kA, vA, oA);
    if (DEPTH > 1 && nchp < 2 && NJ > 1) fetchJ(1, kB, vB, oB);
    int cur = 0;  // the head being multiplied (busy waves)
    // at the first chunk of the next head: the current head's rows out, the
    // next head's queries and own key in (before the chunk fetch that
    // follows, so that their wait does not cover it)
    auto enter = [&](int J) {
      const int hh = J / nch;
      if (hh != cur) {
        close_head(cur);
        cur = hh;
        load_q(h0 + hh);
        open_head(hh);
        // every access of this path done (vmcnt(0), a wait the compiler's
        // own wait insertion sees): otherwise its loads and stores count as
        // pending on the path without a switch too, and the chunk loop waits
        // for every chunk in flight before each fetch
        __builtin_amdgcn_s_waitcnt(0x0f70);
      }
    };
    // Chunk J is multiplied from LDS buffer J % 2 while chunk J + 1 is staged
    // into the other (one barrier per chunk); register sets hold the chunks
    // fetched ahead (DEPTH = 2: chunk c in kA/vA for even c, kB/vB for odd).
    if (NJ > 0) {
      stage(kA, vA, oA, 0);
      fetchJ(min(DEPTH, NJ - 1), kA, vA, oA);  // chunk 2 (DEPTH = 1: chunk 1)
    }
    if constexpr (DEPTH > 1) {
      for (int J = 0; J < NJ; J += 2) {
        __syncthreads();  // buffer 0 holds chunk J; every wave is done with buffer 1
        stage(kB, vB, oB, 1);  // chunk J + 1 (past the last: never read)
        if (wave_busy) enter(J);
        fetchJ(min(J + 3, NJ - 1), kB, vB, oB);
        if (wave_busy) compute(J - cur * nch, nchp, 0);
        if (J + 1 >= NJ) break;
        __syncthreads();
        stage(kA, vA, oA, 0);  // chunk J + 2
        if (wave_busy) enter(J + 1);
        fetchJ(min(J + 4, NJ - 1), kA, vA, oA);
        if (wave_busy) compute(J + 1 - cur * nch, nchp, 1);
      }
    } else {
      for (int J = 0; J < NJ; J += 2) {
        __syncthreads();
        stage(kA, vA, oA, 1);  // chunk J + 1
        if (wave_busy) enter(J);
        fetchJ(min(J + 2, NJ - 1), kA, vA, oA);
        if (wave_busy) compute(J - cur * nch, nchp, 0);
        if (J + 1 >= NJ) break;
        __syncthreads();
        stage(kA, vA, oA, 0);  // chunk J + 2
        if (wave_busy) enter(J + 1);
        fetchJ(min(J + 3, NJ - 1), kA, vA, oA);
        if (wave_busy) compute(J + 1 - cur * nch, nchp, 1);
      }
    }
    if (wave_busy) {  // no chunks (nch = 0): the heads' own keys alone
      close_head(cur);
      for (int hh = cur + 1; hh < hg; ++hh) {
        load_q(h0 + hh);
        open_head(hh);
        close_head(hh);
      }
    }
  } else {
    for (int eb = 0; eb < a.max_extra || eb == 0; eb += TREE_EB) {
      const int ncols = build_columns(eb);
      const int ncp = eb == 0 ? nchp : 0;  // prefix chunks go with the first batch
      const int nch = ncp + (ncols + 63) / 64;
      if (ncp < 1 && nch > 0) fetch(hbase(0), 0, ncp, kA, vA, oA);
      if constexpr (DEPTH > 1) {
        if (ncp < 2 && nch > 1) fetch(hbase(0), 1, ncp, kB, vB, oB);
        for (int j = 0; j < nch; j += 2) {
          __syncthreads();  // every wave is done with the previous chunk
          stage(kA, vA, oA);
          __syncthreads();
          fetch(hbase(0), min(j + 2, nch - 1), ncp, kA, vA, oA);  // past the last: a re-read never staged
          if (wave_busy) compute(j, ncp);
          if (j + 1 >= nch) break;
          __syncthreads();
          stage(kB, vB, oB);
          __syncthreads();
          fetch(hbase(0), min(j + 3, nch - 1), ncp, kB, vB, oB);
          if (wave_busy) compute(j + 1, ncp);
        }
      } else {
        for (int j = 0; j < nch; ++j) {
          __syncthreads();
          stage(kA, vA, oA);
          __syncthreads();
          fetch(hbase(0), min(j + 1, nch - 1), ncp, kA, vA, oA);
          if (wave_busy) compute(j, ncp);
        }
      }
    }
    close_head(0);  // no barriers there
  }
}

// ---------------------------------------------------------------------------
// Groups of at most 16 tokens sharing a prefix (MCTS children of one node):
// one workgroup per (group, head) whose W waves take the prefix's 64-key
// chunks in turn (wave w: chunks w, w + W, ...), so a group's whole prefix
// is requested at once.  A wave holds all of the group's queries in 16x16x32
// MFMAs (S^T = K Q^T: key rows, query columns), loads its chunk's K
// fragments straight into MFMA registers (a lane's key row segment is
// contiguous), stages V in its own LDS tile for the transposing read, and
// keeps its own running max / sum / O.  P enters the PV products rounded to
// bf16 and the row sums unrounded, as in torch's bf16 SDPA.  The waves' partials merge
// through LDS and wave w finishes tokens w, w + W, ... (lane = head dim):
// the private keys (ancestors, then the token itself) and the normalisation.
// Everything a wave needs for its first tokens' private keys is loaded
// before the prefix loop, so those loads overlap the prefix's.
constexpr int FAN_CHUNK = 64, FAN_TILE = FAN_CHUNK * HD;  // bf16 V tile (8 KiB); later the fp32 16 x 64 partial
constexpr int FAN_PT = 2, FAN_PE = 2;  // tokens per wave x private keys per token loaded up front
__device__ const uint4 fan_zero[64] = {};  // read in place of values outside the prefix

// sum over the wave without LDS instructions (DPP within each row of 16
// lanes, then the four rows' lane 0), so it needs no wait on outstanding
// loads into LDS; the result is wave-uniform
ALLIE_DEV float wave_sum_dpp(float v) {
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {  // the control word must be a constant
      case 0x140: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xf, 0xf, false));
      case 0x141: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xf, 0xf, false));
      case 0xb1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xb1, 0xf, 0xf, false));
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4e, 0xf, 0xf, false));
    }
  };
  v += dpp(v, 0x140);  // row_mirror: lane i + lane 15 - i
  v += dpp(v, 0x141);  // row_half_mirror
  v += dpp(v, 0xb1);   // quad_perm [1, 0, 3, 2]
  v += dpp(v, 0x4e);   // quad_perm [2, 3, 0, 1]: every lane holds its row's sum
  const int b = __float_as_int(v);
  return (__int_as_float(__builtin_amdgcn_readlane(b, 0)) + __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
         (__int_as_float(__builtin_amdgcn_readlane(b, 32)) + __int_as_float(__builtin_amdgcn_readlane(b, 48)));
}

ALLIE_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(512, 4) void attn_extend_fan_kernel(ExtendAttnArgs a, int g0) {
  extern __shared__ __attribute__((aligned(1024))) uint16_t fan_lds[];
  const int W = blockDim.x >> 6;
  const int g = g0 + blockIdx.x, head = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lq = lane & 15, lg = lane >> 4;  // MFMA column (query) and lane group
  uint16_t* sV = fan_lds + wave * FAN_TILE;
  float* sML = reinterpret_cast<float*>(fan_lds + W * FAN_TILE);  // [W][m | l][16]
  const int H = a.n_head, d = H * HD, ld = 3 * d;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);
  const bf16_t* __restrict__ pool = reinterpret_cast<const bf16_t*>(a.pool);
  const int64_t voff = (int64_t)H * KV_BLOCK * HD;  // k -> v of the same (block, layer, head)
  const float c2 = a.scale * 1.4426950408889634f;
  const int i0 = a.group_start[g];
  const int nq = a.group_start[g + 1] - i0;  // <= 16
  const int P = a.prefix_len[g];
  const int32_t* btab = a.prefix_blocks + (int64_t)g * a.max_blocks;
  // K rows of (block 0, this layer, this head); a block adds bstride
  const bf16_t* lbase = pool + ((int64_t)a.layer * a.pool_blocks * 2 * H + head) * (KV_BLOCK * HD);
  const int64_t bstride = (int64_t)2 * H * KV_BLOCK * HD;
  auto slot_ok = [&](int sl) { return sl >= 0 && (sl >> 4) < a.pool_blocks; };
  auto slot_off = [&](int sl) { return pool_off(slot_ok(sl) ? sl >> 4 : 0, a.pool_blocks, a.layer, 0, H, head, sl & 15); };
  auto clamp_e = [&](int E) { return E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E); };

  // ---- the wave's first FAN_PT tokens (w + W t): their first FAN_PE private
  // keys load together with the prefix and are folded in (lane = head dim)
  // after it
  int xn[FAN_PT];
  float xm[FAN_PT], xl[FAN_PT], xa[FAN_PT];  // running max (raw score), sum, P V
  uint32_t xq[FAN_PT], xk[FAN_PT][FAN_PE], xv[FAN_PT][FAN_PE];  // raw bf16 (converted where used)
  int xs[FAN_PT][FAN_PE];
#pragma unroll
  for (int t = 0; t < FAN_PT; ++t) {
    const int q = wave + W * t;
    const int i = i0 + (q < nq ? q : 0);
    xn[t] = q < nq ? clamp_e(a.n_extra[i]) : 0;
#pragma unroll
    for (int e = 0; e < FAN_PE; ++e) xs[t][e] = e < a.max_extra ? a.extra_slot[(int64_t)i * a.max_extra + e] : -1;
    xq[t] = qkv[(int64_t)i * ld + head * HD + lane];
  }
  auto fold_extras = [&]() {
#pragma unroll
    for (int t = 0; t < FAN_PT; ++t) {
      float m = -INFINITY, l = 0.f, acc = 0.f;
#pragma unroll
      for (int e = 0; e < FAN_PE; ++e) {
        if (e >= xn[t] || !slot_ok(xs[t][e])) continue;  // uniform
        const float sc = wave_sum_dpp(bf2f(xq[t]) * bf2f(xk[t][e]));  // raw score (scaled in the exponent)
        const float m_new = fmaxf(m, sc);
        const float alpha = __builtin_amdgcn_exp2f((m - m_new) * c2);  // m = -inf: 0
        const float pe = __builtin_amdgcn_exp2f((sc - m_new) * c2);
        l = l * alpha + pe;
        acc = acc * alpha + round_bf16(pe) * bf2f(xv[t][e]);
        m = m_new;
      }
      xm[t] = m;
      xl[t] = l;
      xa[t] = acc;
    }
  };

  const int nch = (max(P, 0) + FAN_CHUNK - 1) / FAN_CHUNK;
  // lane j holds block j % 4 of the wave's chunk j / 4: a wave has at most
  // 16 chunks (FAN_MAX_BLOCKS), so the chunk loop makes no global load of its
  // own (one there would make the compiler's wait before the chunk's loads
  // cover every load issued before them); the table row is read before the
  // prefix length is known
  int bt;
  {
    const int bi = (wave + W * (lane >> 2)) * 4 + (lane & 3);
    const int v = bi < a.max_blocks ? btab[bi] : -1;
    bt = (bi * KV_BLOCK < P && v >= 0 && v < a.pool_blocks) ? v : -1;
  }
  // queries: B operand of S^T = K Q^T, query lq, dims 32 ks + 8 lg .. +7
  const bool q_ok = lq < nq;
  const int qi = i0 + (q_ok ? lq : 0);
  const int lim = q_ok ? min(P, a.pos[qi]) : 0;
  bf16x8_t qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(qkv + (int64_t)qi * ld + head * HD + 32 * ks + 8 * lg));
  // the private keys' rows (their slots are in by now)
#pragma unroll
  for (int t = 0; t < FAN_PT; ++t)
#pragma unroll
    for (int e = 0; e < FAN_PE; ++e) {
      const int64_t kb = slot_off(xs[t][e]) + lane;
      xk[t][e] = pool[kb];
      xv[t][e] = pool[kb + voff];
    }
  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t o[4] = {f32x4_t{}, f32x4_t{}, f32x4_t{}, f32x4_t{}};  // O^T: dims 16 db + 4 lg .. +3 of query lq
  for (int c = wave, n = 0; c < nch; c += W, ++n) {
    const int k0 = c * FAN_CHUNK;
    // the chunk's 4 pool blocks (wave-uniform)
    int blk[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      blk[b] = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(bt, 4 * n + b));
    // V rows by DMA: instruction t, lane i fills row r = 8 t + i / 8 at
    // 16-byte position i % 8 (chunk (i % 8) ^ (2 ((r >> 1) & 1)); the swizzle
    // bit of r comes from i alone), from block t / 2; rows past the prefix or
    // in a skipped block read zeros
    {
      const int rr = lane >> 3;
      const int vlo = rr * HD + (((lane & 7) ^ (((rr >> 1) & 1) << 1)) << 3);  // elements
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int b = t >> 1, r = 8 * t + rr;
        const bf16_t* vb = lbase + (int64_t)max(blk[b], 0) * bstride + voff + (t & 1) * 8 * HD;
        const bool vok = blk[b] >= 0 && k0 + r < P;
        const void* src = vok ? (const void*)(vb + vlo) : (const void*)(reinterpret_cast<const bf16_t*>(fan_zero) + vlo);
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(sV + t * 512), 16, 0, 0);
      }
    }
    // K fragments (key 16 kb + lq, dims 32 ks + 8 lg .. +7) into registers;
    // keys of a skipped block read block 0 and are masked
    u32x4_t kf[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const bf16_t* kr = lbase + (int64_t)max(blk[kb], 0) * bstride + lq * HD + 8 * lg;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) kf[kb][ks] = *(const __attribute__((address_space(1))) u32x4_t*)(kr + 32 * ks);
    }
    f32x4_t st[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      st[kb] = f32x4_t{};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[kb][ks]), qf[ks], st[kb], 0, 0, 0);
    }
    // st[kb][r]: key 16 kb + 4 lg + r of query lq; keys past the query's
    // limit or in a skipped block are masked
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (k0 + 16 * kb + 4 * lg + r >= lim || blk[kb] < 0) st[kb][r] = -INFINITY;
        mx = fmaxf(mx, st[kb][r]);
      }
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    u32x4_t pf[2];  // P^T of k-step s: keys 32 s + 4 lg + {0..3}, then 32 s + 16 + 4 lg + {0..3}
    if (m_new != -INFINITY) {  // uniform per query
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c2);
      m_run = m_new;
      const float mc = m_new * c2;
      float p[4][4];
      float ls = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kb][r] = __builtin_amdgcn_exp2f(fmaf(st[kb][r], c2, -mc));
          ls += p[kb][r];
        }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        pf[s2] = u32x4_t{pack_bf16x2(p[2 * s2][0], p[2 * s2][1]), pack_bf16x2(p[2 * s2][2], p[2 * s2][3]),
                         pack_bf16x2(p[2 * s2 + 1][0], p[2 * s2 + 1][1]), pack_bf16x2(p[2 * s2 + 1][2], p[2 * s2 + 1][3])};
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    } else {
      pf[0] = pf[1] = u32x4_t{0, 0, 0, 0};
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the tile's DMA is done
    wave_lds_sync();
    // O^T += V^T P^T: A = V^T rows (dims 16 db + lq), k-slots as P^T's,
    // read transposed: lane group lg reads keys 32 s + 4 lg + (lq >> 2) (and
    // + 16)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int r0 = 32 * s2 + 4 * lg + (lq >> 2), r1 = r0 + 16;
        const int j = 4 * db + (lq & 3);
        const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r0 * HD + ((j ^ (((r0 >> 1) & 1) << 2)) << 2)));
        const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r1 * HD + ((j ^ (((r1 >> 1) & 1) << 2)) << 2)));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, u32x4_t{l2.x, l2.y, h2.x, h2.y}),
                                                        __builtin_bit_cast(bf16x8_t, pf[s2]), o[db], 0, 0, 0);
      }
    wave_lds_sync();  // the transposing reads are done before the tile is written again
  }
  fold_extras();  // their loads went out with the prefix's
  // ---- the wave's partial to LDS: O as fp32 [query][64 dims], 16-byte
  // group j of row q at j ^ q; running max and sum per query -----------------
  float* so = reinterpret_cast<float*>(sV);
#pragma unroll
  for (int db = 0; db < 4; ++db)
    *reinterpret_cast<f32x4_t*>(so + lq * HD + (((4 * db + lg) ^ lq) << 2)) = o[db];
  const float l_tot = xor32_sum(xor16_sum(l_run));
  if (lg == 0) {
    sML[wave * 32 + lq] = m_run;
    sML[wave * 32 + 16 + lq] = l_tot;
  }
  __syncthreads();
  // ---- wave w finishes tokens w, w + W, ... (lane = head dim): merges the
  // waves' partials with the token's folded private keys, then its
  // remaining private keys from e0 on, and normalises -------------------------
  auto finish = [&](int q, int E, int e0, float m, float l, float acc) {
    const int i = i0 + q;
    float mp = -INFINITY;
    for (int w = 0; w < W; ++w) mp = fmaxf(mp, sML[w * 32 + q]);
    if (mp != -INFINITY) {
      const float mt = fmaxf(m, mp);
      const float f0 = __builtin_amdgcn_exp2f((m - mt) * c2);  // m = -inf: 0
      l *= f0;
      acc *= f0;
      for (int w = 0; w < W; ++w) {
        const float mw = sML[w * 32 + q];
        if (mw == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f((mw - mt) * c2);
        l += f * sML[w * 32 + 16 + q];
        acc += f * reinterpret_cast<const float*>(fan_lds + w * FAN_TILE)[q * HD + (((lane >> 2) ^ q) << 2) + (lane & 3)];
      }
      m = mt;
    }
    if (e0 < E) {
      const float qv = bf2f(qkv[(int64_t)i * ld + head * HD + lane]);
      for (int e = e0; e < E; ++e) {
        const int sl = a.extra_slot[(int64_t)i * a.max_extra + e];
        if (!slot_ok(sl)) continue;
        const int64_t kb = slot_off(sl) + lane;
        const float sc = wave_sum(qv * bf2f(pool[kb]));
        const float m_new = fmaxf(m, sc);
        const float alpha = __builtin_amdgcn_exp2f((m - m_new) * c2);
        const float pe = __builtin_amdgcn_exp2f((sc - m_new) * c2);
        l = l * alpha + pe;
        acc = acc * alpha + round_bf16(pe) * bf2f(pool[kb + voff]);
        m = m_new;
      }
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    reinterpret_cast<bf16_t*>(a.out)[(int64_t)i * d + head * HD + lane] = (bf16_t)f2bf(acc * inv);
  };
#pragma unroll
  for (int t = 0; t < FAN_PT; ++t) {
    const int q = wave + W * t;
    if (q < nq) finish(q, xn[t], FAN_PE, xm[t], xl[t], xa[t]);
  }
  for (int q = wave + W * FAN_PT; q < nq; q += W) finish(q, clamp_e(a.n_extra[i0 + q]), 0, -INFINITY, 0.f, 0.f);
}

}  // namespace

namespace allie {

hipError_t launch_extend_prepare(const ExtendPrepArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(extend_prepare_kernel, dim3(1), dim3(PREP_THREADS), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_extend_tiles(const int32_t* group_start, int first_group, int n_groups, int tile_q, int32_t* tiles,
                               hipStream_t st) {
  if (first_group >= n_groups) return hipSuccess;
  if (tile_q <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(extend_tiles_kernel, dim3(1), dim3(PREP_THREADS), 0, st, group_start, first_group, n_groups,
                     tile_q, tiles);
  return hipGetLastError();
}

hipError_t launch_decode_order(const ExtendAttnArgs& a, int n, int32_t* order, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (!order) return hipErrorInvalidValue;
  hipLaunchKernelGGL(decode_order_kernel, dim3(1), dim3(PREP_THREADS), 0, st, a, n, order);
  return hipGetLastError();
}

hipError_t launch_attn_extend_wave(const ExtendAttnArgs& a, hipStream_t st) {
  const int64_t waves = (int64_t)a.n * a.n_head;
  if (waves == 0) return hipSuccess;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (a.act_bf16)
    launch_timed(attn_extend_wave_kernel<bf16_t>, grid, dim3(256), 0, st, a);
  else
    launch_timed(attn_extend_wave_kernel<float>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_attn_extend_split(const ExtendAttnArgs& a, hipStream_t st) {
  if (!a.act_bf16) return hipErrorInvalidValue;
  const int64_t rows = (int64_t)a.n * a.n_head;
  if (rows == 0) return hipSuccess;
  if (rows > DECODE_SPLIT_MAX_ROWS) return hipErrorInvalidValue;
  launch_timed(attn_extend_split_kernel<8>, dim3((unsigned)rows), dim3(8 * 64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_attn_extend_fan(const ExtendAttnArgs& a, int g0, int g1, int waves, hipStream_t st) {
  if (!a.act_bf16 || g1 > a.n_groups || waves > 8) return hipErrorInvalidValue;
  const int W = waves > 0 ? waves : fan_waves(a.max_blocks);
  if ((a.max_blocks + 3) / 4 > 16 * W) return hipErrorInvalidValue;  // a wave's chunks: at most 16
  const size_t lds = (size_t)W * (FAN_TILE * 2 + 32 * 4);
  if (g1 > g0) launch_timed(attn_extend_fan_kernel, dim3(g1 - g0, a.n_head), dim3(64 * W), (uint32_t)lds, st, a, g0);
  return hipGetLastError();
}

constexpr int TREE_MIN_WG = 1024;  // two rounds of two 8-wave workgroups per CU
// Heads per tree workgroup (one column batch only, else 1): the caller's
// a.head_group when it divides the head count; for 0, on 128-query tiles,
// the largest of 16, 8, 4, 2 that divides it and still leaves at least
// TREE_MIN_WG workgroups; else 1.  (The 64-query, one-chunk-in-registers
// instance with several heads spills registers, so 0 keeps those tiles at
// one head; it runs only when a caller asks for it.)
int tree_head_group(const ExtendAttnArgs& a) {
  if (a.max_extra > TREE_EB) return 1;
  if (a.head_group > 0) return a.n_head % a.head_group == 0 ? a.head_group : 1;
  if (a.tile_q != 128) return 1;
  for (int hg = 16; hg > 1; hg >>= 1)
    if (a.n_head % hg == 0 && (int64_t)a.n_tiles * (a.n_head / hg) >= TREE_MIN_WG) return hg;
  return 1;
}

hipError_t launch_attn_extend_tree(const ExtendAttnArgs& a0, hipStream_t st) {
  if (!a0.self_slot || a0.max_blocks > TREE_MAX_BLOCKS) return hipErrorInvalidValue;
  if (!a0.act_bf16 || a0.tiles == nullptr) return hipErrorInvalidValue;
  if (a0.n_tiles == 0) return hipSuccess;
  ExtendAttnArgs a = a0;
  a.head_group = tree_head_group(a0);
  const dim3 grid(a.n_tiles, a.n_head / a.head_group);
  const bool mh = a.head_group > 1;
  if (a.tile_q == 128) {  // 8 waves, two chunks in flight
    if (mh)
      launch_timed(attn_extend_tree_kernel<8, 2, true>, grid, dim3(512), 0, st, a);
    else
      launch_timed(attn_extend_tree_kernel<8, 2, false>, grid, dim3(512), 0, st, a);
  } else if (a.tile_q == 64) {  // 4 waves, one chunk in flight (registers)
    if (mh)
      launch_timed(attn_extend_tree_kernel<4, 1, true>, grid, dim3(256), 0, st, a);
    else
      launch_timed(attn_extend_tree_kernel<4, 1, false>, grid, dim3(256), 0, st, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace allie
