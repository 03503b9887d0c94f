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
// Pool layout (one block = 16 positions of every layer):
//   [block][layer][k|v][head][16][64]  (bf16, or fp32 in the fp32 check mode)
// so one (block, layer, k|v, head) is a contiguous 2 KiB (bf16) row group.
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
constexpr int QT = 64;           // queries per tree-kernel tile
constexpr int KT = 64;           // prefix keys per LDS tile (4 pool blocks)
constexpr int PREP_THREADS = 1024;

// element offset of (block, layer, k|v, head, offset-in-block, dim 0)
ALLIE_DEV int64_t pool_off(int64_t blk, int L, int layer, int kv, int H, int head, int off) {
  return ((((blk * L + layer) * 2 + kv) * H + head) * KV_BLOCK + off) * (int64_t)HD;
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

// Tile list of the tree kernel: (g << 8) | t for t < ceil(size_g / 64), groups
// in order.  One workgroup; exclusive scan of the per-group tile counts.
__global__ __launch_bounds__(PREP_THREADS) void extend_tiles_kernel(const int32_t* __restrict__ group_start,
                                                                    int g0, int G, int32_t* __restrict__ tiles) {
  __shared__ int sh[PREP_THREADS / 64 + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int carry = 0;
  for (int base = g0; base < G; base += PREP_THREADS) {
    const int g = base + threadIdx.x;
    const int nt = g < G ? (group_start[g + 1] - group_start[g] + QT - 1) / QT : 0;
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

template <typename T>
__global__ __launch_bounds__(256) void attn_extend_wave_kernel(ExtendAttnArgs a) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int H = a.n_head, d = H * HD;
  if (wid >= (int64_t)a.n * H) return;  // no barriers below: whole waves leave
  const int i = (int)(wid / H), head = (int)(wid % H);
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
  auto locate = [&](int c, int64_t& off, bool& ok) {
    int blk, kpos;
    if (c < nbp) {
      blk = c < 64 ? __builtin_amdgcn_readlane(my_blk, c) : btab[c];
      kpos = kj;
      ok = c * KV_BLOCK + kj < P;
    } else {
      const int e = (c - nbp) * KV_BLOCK + kj;
      const int sl = e < E ? a.extra_slot[(int64_t)i * a.max_extra + e] : -1;
      blk = sl >> 4;
      kpos = sl & 15;
      ok = sl >= 0;
    }
    ok = ok && blk >= 0 && blk < a.pool_blocks;
    off = pool_off(ok ? blk : 0, a.n_layer, a.layer, 0, H, head, ok ? kpos : 0) + dq;
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
    s += __shfl_xor(s, 1, 64);  // the 4 lanes of a key share ok
    s += __shfl_xor(s, 2, 64);
    s = ok ? s : -INFINITY;
    float mb = s;
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) mb = fmaxf(mb, __shfl_xor(mb, o, 64));
    const float m_new = fmaxf(m_run, mb);
    if (m_new == -INFINITY) return;  // nothing visible yet (wave-uniform)
    const float alpha = exp2f(m_run - m_new);
    const float p = ok ? exp2f(s - m_new) : 0.f;
    l_run = l_run * alpha + ((lane & 3) == 0 ? p : 0.f);
    float vv[16];
    widen16<T>(vr, vv);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = acc[j] * alpha + p * vv[j];
    m_run = m_new;
  };
  auto fetch_chunk = [&](int c, Row16<T>& kr, Row16<T>& vr, bool& ok) {
    int64_t off;
    locate(c, off, ok);
    fetch16<T>(pool + off, kr);
    fetch16<T>(pool + off + voff, vr);
  };
  // two register buffers: chunk c + 1 loads while chunk c is reduced
  Row16<T> kA, vA, kB, vB;
  bool okA = false, okB = false;
  if (nch > 0) fetch_chunk(0, kA, vA, okA);
  for (int c = 0; c < nch; c += 2) {
    if (c + 1 < nch) fetch_chunk(c + 1, kB, vB, okB);
    reduce_chunk(kA, vA, okA);
    if (c + 1 >= nch) break;
    if (c + 2 < nch) fetch_chunk(c + 2, kA, vA, okA);
    reduce_chunk(kB, vB, okB);
  }
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

// ---------------------------------------------------------------------------
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x4_ll __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_ll lds_f16x4_t;

// two fp32 -> packed fp16 (round toward zero: exact for bf16 inputs in range)
ALLIE_DEV uint32_t pk_f16(float a, float b) { return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b)); }

__global__ __launch_bounds__(128) void attn_extend_tree_kernel(ExtendAttnArgs a) {
  // K rows of 128 B: 16-byte chunk c of row r at c ^ ((r >> 1) & 7).  V rows
  // (converted to fp16) of 128 B: 8-byte chunk j of row r at
  // j ^ (4 ((r >> 1) & 1)), read transposed (ds_read_b64_tr_b16) as in the
  // varlen prefill kernel.
  __shared__ __attribute__((aligned(1024))) uint16_t sK[KT * HD];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[KT * HD];

  const int head = blockIdx.y;
  const int tile = a.tiles[blockIdx.x];
  const int g = tile >> 8, qt = tile & 255;
  const int H = a.n_head, d = H * HD, ld = 3 * d;
  const int q_end = a.group_start[g + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = lane >> 5, ql = lane & 31;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);
  const bf16_t* __restrict__ pool = reinterpret_cast<const bf16_t*>(a.pool);

  const int q_first = a.group_start[g] + qt * QT;
  const int qi = q_first + wave * 32 + ql;
  const bool q_ok = qi < q_end;
  // a wave whose 32 queries are all past the group computes nothing (it
  // still stages its share of the keys)
  const bool wave_busy = q_first + wave * 32 < q_end;
  bf16x8_t qf[4];  // B operand of S^T = K Q^T: head dims 16 kk + 8 hf .. +7
  {
    const bf16_t* qrow = qkv + (int64_t)(q_ok ? qi : 0) * ld + head * HD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4_t v = q_ok ? *reinterpret_cast<const u32x4_t*>(qrow + kk * 16 + hf * 8) : u32x4_t{0, 0, 0, 0};
      qf[kk] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  const float c2 = a.scale * 1.4426950408889634f;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};

  // ---- phase 1: the group's prefix, 64 keys (4 pool blocks) per LDS tile;
  // the next tile's keys and values load into registers while one is
  // multiplied.  Query qi sees prefix positions below lim (its own position
  // when that is inside the prefix: the tokens of a new game's prefix).
  const int P = a.prefix_len[g];
  const int lim = q_ok ? min(P, a.pos[qi]) : 0;
  const int32_t* btab = a.prefix_blocks + (int64_t)g * a.max_blocks;
  // thread's 4 chunks of a tile: key (tid + 128 it) / 8, 16-byte chunk % 8
  uint4 kv[4], vv[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int cidx = tid + 128 * it;
      const int key = cidx >> 3, c = cidx & 7;
      const int p = k0 + key;
      const int bi = p / KV_BLOCK;
      const int blk = (p < P && bi < a.max_blocks) ? btab[bi] : -1;
      kv[it] = make_uint4(0, 0, 0, 0);
      vv[it] = make_uint4(0, 0, 0, 0);
      if (blk >= 0 && blk < a.pool_blocks) {
        const int64_t base = pool_off(blk, a.n_layer, a.layer, 0, H, head, p % KV_BLOCK) + c * 8;
        kv[it] = *reinterpret_cast<const uint4*>(pool + base);
        vv[it] = *reinterpret_cast<const uint4*>(pool + base + (int64_t)H * KV_BLOCK * HD);  // k -> v
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int cidx = tid + 128 * it;
      const int key = cidx >> 3, c = cidx & 7;
      *reinterpret_cast<uint4*>(sK + key * HD + ((c ^ ((key >> 1) & 7)) << 3)) = kv[it];
      uint4 h;
      h.x = pk_f16(bf2f(vv[it].x & 0xffffu), bf2f(vv[it].x >> 16));
      h.y = pk_f16(bf2f(vv[it].y & 0xffffu), bf2f(vv[it].y >> 16));
      h.z = pk_f16(bf2f(vv[it].z & 0xffffu), bf2f(vv[it].z >> 16));
      h.w = pk_f16(bf2f(vv[it].w & 0xffffu), bf2f(vv[it].w >> 16));
      *reinterpret_cast<uint4*>(sV + key * HD + ((c ^ (((key >> 1) & 1) << 1)) << 3)) = h;
    }
  };
  // transposing V read of lane l: row (l % 16) / 4 of a 4-key group, dims
  // 16 ((l / 16) % 2) + 4 (l % 4) .. + 3 of a 32-dim block
  const int trow = (lane & 15) >> 2;
  const int tchunk = ((lane >> 4) & 1) * 4 + (lane & 3);
  if (P > 0) fetch(0);
  for (int k0 = 0; k0 < P; k0 += KT) {
    __syncthreads();  // every wave is done with the previous tile
    stage();
    __syncthreads();
    if (k0 + KT < P) fetch(k0 + KT);
    if (!wave_busy) continue;
    f32x16_t st[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      st[b] = f32x16_t{};
      const int krow = b * 32 + ql;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8_t kf = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(sK + krow * HD + (((2 * kk + hf) ^ ((krow >> 1) & 7)) << 3)));
        st[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], st[b], 0, 0, 0);
      }
    }
    // keys past the query's limit or in a skipped block are masked
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int p = k0 + b * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        const int bi = p / KV_BLOCK;
        const int blk = (p < P && bi < a.max_blocks) ? btab[bi] : -1;
        if (blk < 0 || blk >= a.pool_blocks || p >= lim) st[b][r] = -INFINITY;
        mx = fmaxf(mx, st[b][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    uint32_t pk[2][8];
    if (m_new != -INFINITY) {  // uniform per query (both lanes of a query agree)
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c2);
      m_run = m_new;
      const float mc = m_new * c2;
      float ls = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(st[b][r], c2, -mc));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(st[b][r + 1], c2, -mc));
          ls += p0 + p1;
          pk[b][r >> 1] = pk_f16(p0, p1);
        }
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[hb][r] *= alpha;
    } else {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 8; ++r) pk[b][r] = 0u;
    }
    // O^T += V^T P^T: k-step (b, mm) covers keys 32 b + 16 mm + {4 hf .. +3,
    // 8 + 4 hf .. +3} (the S^T layout), identically for V^T
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        const f16x8_t pf = __builtin_bit_cast(
            f16x8_t, u32x4_t{pk[b][4 * mm], pk[b][4 * mm + 1], pk[b][4 * mm + 2], pk[b][4 * mm + 3]});
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const int r0 = b * 32 + 16 * mm + 4 * hf + trow, r1 = r0 + 8;
          const int j = hb * 8 + tchunk;
          const fp16x4_ll lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
              (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r0 * HD + ((j ^ (((r0 >> 1) & 1) << 2)) << 2)));
          const fp16x4_ll hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
              (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r1 * HD + ((j ^ (((r1 >> 1) & 1) << 2)) << 2)));
          const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
          const f16x8_t vf = __builtin_bit_cast(f16x8_t, u32x4_t{l2.x, l2.y, h2.x, h2.y});
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[hb], 0, 0, 0);
        }
      }
  }
  if (!q_ok) return;  // no barriers below

  // ---- phase 2: the query's private keys (ancestors, then itself) -----------
  // lanes l and l ^ 32 share query qi: each holds half of q (dims 16 kk + 8 hf
  // + [0, 8)) and half of o (dims 32 hb + 8 q4 + 4 hf + [0, 4)).
  int E = a.n_extra[qi];
  E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
  for (int e = 0; e < E; ++e) {
    const int sl = a.extra_slot[(int64_t)qi * a.max_extra + e];
    if (sl < 0 || (sl >> 4) >= a.pool_blocks) continue;  // same decision in both lanes
    const int64_t kb = pool_off(sl >> 4, a.n_layer, a.layer, 0, H, head, sl & 15);
    float s = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(pool + kb + kk * 16 + hf * 8);
      const u32x4_t qw = __builtin_bit_cast(u32x4_t, qf[kk]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s = fmaf(bf2f(qw[t] & 0xffffu), bf2f(kw[t] & 0xffffu), s);
        s = fmaf(bf2f(qw[t] >> 16), bf2f(kw[t] >> 16), s);
      }
    }
    s = s + __shfl_xor(s, 32, 64);  // raw score, as m_run (scaled in the exponent)
    const float m_new = fmaxf(m_run, s);
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c2);
    const float p = __builtin_amdgcn_exp2f((s - m_new) * c2);
    l_run = l_run * alpha + (hf == 0 ? p : 0.f);
    const int64_t vb = kb + (int64_t)H * KV_BLOCK * HD;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const u32x2_t vw = *reinterpret_cast<const u32x2_t*>(pool + vb + hb * 32 + q4 * 8 + 4 * hf);
        o[hb][q4 * 4 + 0] = o[hb][q4 * 4 + 0] * alpha + p * bf2f(vw.x & 0xffffu);
        o[hb][q4 * 4 + 1] = o[hb][q4 * 4 + 1] * alpha + p * bf2f(vw.x >> 16);
        o[hb][q4 * 4 + 2] = o[hb][q4 * 4 + 2] * alpha + p * bf2f(vw.y & 0xffffu);
        o[hb][q4 * 4 + 3] = o[hb][q4 * 4 + 3] * alpha + p * bf2f(vw.y >> 16);
      }
    m_run = m_new;
  }
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  bf16_t* out = reinterpret_cast<bf16_t*>(a.out) + (int64_t)qi * d + head * HD;
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int hd = hb * 32 + q4 * 8 + 4 * hf;
      uint2 p;
      p.x = pack_bf16x2(o[hb][q4 * 4 + 0] * inv, o[hb][q4 * 4 + 1] * inv);
      p.y = pack_bf16x2(o[hb][q4 * 4 + 2] * inv, o[hb][q4 * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(out + hd) = p;
    }
}

// ---------------------------------------------------------------------------
// Groups of at most 32 tokens sharing a prefix (MCTS children of one node):
// one workgroup per (group, head) whose W waves take the prefix's 64-key
// chunks in turn (wave w: chunks w, w + W, ...), so the prefix is read by W
// chunks at once rather than one tile after another.  A wave holds all of
// the group's queries (S^T = K Q^T, 32 query columns), loads its chunk's K
// fragments straight into MFMA registers (a lane's key row is contiguous),
// stages V as fp16 in its own LDS tile for the transposing read, and keeps
// its own running max / sum / O.  The waves' partials then merge through LDS
// and wave w finishes tokens w, w + W, ... (lane = head dim): the private
// keys (ancestors, then the token itself) and the normalisation.
constexpr int FAN_CHUNK = 64, FAN_TILE = FAN_CHUNK * HD;  // fp16 V tile = fp32 32 x 64 partial, 8 KiB

ALLIE_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(512) void attn_extend_fan_kernel(ExtendAttnArgs a, int g0) {
  extern __shared__ __attribute__((aligned(1024))) uint16_t fan_lds[];
  const int W = blockDim.x >> 6;
  const int g = g0 + blockIdx.x, head = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ql = lane & 31, hf = lane >> 5;
  uint16_t* sV = fan_lds + wave * FAN_TILE;  // V tile (fp16, rows as in the tree kernel); then O partial
  float* sML = reinterpret_cast<float*>(fan_lds + W * FAN_TILE);  // [W][m | l][32]
  const int H = a.n_head, d = H * HD, ld = 3 * d;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);
  const bf16_t* __restrict__ pool = reinterpret_cast<const bf16_t*>(a.pool);
  const int i0 = a.group_start[g];
  const int nq = a.group_start[g + 1] - i0;  // <= 32
  const int qi = i0 + ql;
  const bool q_ok = ql < nq;
  const int P = a.prefix_len[g];
  const int lim = q_ok ? min(P, a.pos[qi]) : 0;
  const int32_t* btab = a.prefix_blocks + (int64_t)g * a.max_blocks;
  auto block_of = [&](int p) {
    const int bi = p / KV_BLOCK;
    const int blk = (p < P && bi < a.max_blocks) ? btab[bi] : -1;
    return (blk >= 0 && blk < a.pool_blocks) ? blk : -1;
  };
  const int64_t voff = (int64_t)H * KV_BLOCK * HD;  // k -> v of the same (block, layer, head)
  bf16x8_t qf[4];  // B operand: head dims 16 kk + 8 hf .. +7 of query ql
  {
    const bf16_t* qrow = qkv + (int64_t)(q_ok ? qi : i0) * ld + head * HD + hf * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(qrow + kk * 16));
  }
  const float c2 = a.scale * 1.4426950408889634f;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};
  const int trow = (lane & 15) >> 2;
  const int tchunk = ((lane >> 4) & 1) * 4 + (lane & 3);
  const int nch = (max(P, 0) + FAN_CHUNK - 1) / FAN_CHUNK;
  for (int c = wave; c < nch; c += W) {
    const int k0 = c * FAN_CHUNK;
    // loads of the chunk: the V row of key `lane` (8 x 16 bytes), then K
    // fragments (key 32 b + ql, dims 16 kk + 8 hf .. +7).  A key outside a
    // valid block reads block 0 and is zeroed (V) or masked (K).
    const int vblk = block_of(k0 + lane);
    const uint64_t ok = __ballot(vblk >= 0);  // bit = key - k0
    uint4 vv[8];
    {
      const bf16_t* vr = pool + pool_off(vblk >= 0 ? vblk : 0, a.n_layer, a.layer, 0, H, head, (k0 + lane) % KV_BLOCK) + voff;
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) vv[ch] = *reinterpret_cast<const uint4*>(vr + ch * 8);
    }
    u32x4_t kf[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int p = k0 + b * 32 + ql;
      const int blk = block_of(p);
      const bf16_t* kr = pool + pool_off(blk >= 0 ? blk : 0, a.n_layer, a.layer, 0, H, head, p % KV_BLOCK) + hf * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) kf[b][kk] = *reinterpret_cast<const u32x4_t*>(kr + kk * 16);
    }
    // V row `lane` to the wave's tile as fp16 (8-byte chunk j of row r at
    // j ^ (4 ((r >> 1) & 1)))
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      const uint4 v = vblk >= 0 ? vv[ch] : make_uint4(0, 0, 0, 0);
      uint4 h;
      h.x = pk_f16(bf2f(v.x & 0xffffu), bf2f(v.x >> 16));
      h.y = pk_f16(bf2f(v.y & 0xffffu), bf2f(v.y >> 16));
      h.z = pk_f16(bf2f(v.z & 0xffffu), bf2f(v.z >> 16));
      h.w = pk_f16(bf2f(v.w & 0xffffu), bf2f(v.w >> 16));
      *reinterpret_cast<uint4*>(sV + lane * HD + ((ch ^ (((lane >> 1) & 1) << 1)) << 3)) = h;
    }
    __builtin_amdgcn_sched_barrier(0);  // V registers free before the products
    f32x16_t st[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      st[b] = f32x16_t{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        st[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[b][kk]), qf[kk], st[b], 0, 0, 0);
    }
    // keys past the query's limit or in a skipped block are masked
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kl = b * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (k0 + kl >= lim || !((ok >> kl) & 1)) st[b][r] = -INFINITY;
        mx = fmaxf(mx, st[b][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    uint32_t pk[2][8];
    if (m_new != -INFINITY) {  // uniform per query (both lanes of a query agree)
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c2);
      m_run = m_new;
      const float mc = m_new * c2;
      float ls = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(st[b][r], c2, -mc));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(st[b][r + 1], c2, -mc));
          ls += p0 + p1;
          pk[b][r >> 1] = pk_f16(p0, p1);
        }
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[hb][r] *= alpha;
    } else {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 8; ++r) pk[b][r] = 0u;
    }
    wave_lds_sync();  // the tile's V rows are written
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        const f16x8_t pf = __builtin_bit_cast(
            f16x8_t, u32x4_t{pk[b][4 * mm], pk[b][4 * mm + 1], pk[b][4 * mm + 2], pk[b][4 * mm + 3]});
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const int r0 = b * 32 + 16 * mm + 4 * hf + trow, r1 = r0 + 8;
          const int j = hb * 8 + tchunk;
          const fp16x4_ll lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
              (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r0 * HD + ((j ^ (((r0 >> 1) & 1) << 2)) << 2)));
          const fp16x4_ll hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
              (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r1 * HD + ((j ^ (((r1 >> 1) & 1) << 2)) << 2)));
          const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(f16x8_t, u32x4_t{l2.x, l2.y, h2.x, h2.y}), pf, o[hb], 0, 0, 0);
        }
      }
    wave_lds_sync();  // the transposing reads are done before the next tile's writes
  }
  // ---- the wave's partial to LDS: O as fp32 [query][64 dims], 16-byte
  // group j of row q at j ^ (q & 15); running max and sum per query ---------
  float* so = reinterpret_cast<float*>(sV);
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int j = hb * 8 + q4 * 2 + hf;  // dims 4 j .. 4 j + 3
      *reinterpret_cast<float4*>(so + ql * HD + ((j ^ (ql & 15)) << 2)) =
          make_float4(o[hb][q4 * 4 + 0], o[hb][q4 * 4 + 1], o[hb][q4 * 4 + 2], o[hb][q4 * 4 + 3]);
    }
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (hf == 0) {
    sML[wave * 64 + ql] = m_run;
    sML[wave * 64 + 32 + ql] = l_tot;
  }
  __syncthreads();
  // ---- wave w finishes tokens w, w + W, ... (lane = head dim) -------------
  for (int q = wave; q < nq; q += W) {
    const int i = i0 + q;
    float m = -INFINITY;
    for (int w = 0; w < W; ++w) m = fmaxf(m, sML[w * 64 + q]);
    float l = 0.f, acc = 0.f;
    for (int w = 0; w < W; ++w) {
      const float mw = sML[w * 64 + q];
      if (mw == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f((mw - m) * c2);
      l += f * sML[w * 64 + 32 + q];
      acc += f * reinterpret_cast<const float*>(fan_lds + w * FAN_TILE)[q * HD + (((lane >> 2) ^ (q & 15)) << 2) + (lane & 3)];
    }
    const float qv = bf2f(qkv[(int64_t)i * ld + head * HD + lane]);
    int E = a.n_extra[i];
    E = E < 0 ? 0 : (E > a.max_extra ? a.max_extra : E);
    for (int e = 0; e < E; ++e) {
      const int sl = a.extra_slot[(int64_t)i * a.max_extra + e];
      if (sl < 0 || (sl >> 4) >= a.pool_blocks) continue;
      const int64_t kb = pool_off(sl >> 4, a.n_layer, a.layer, 0, H, head, sl & 15);
      const float kv = bf2f(pool[kb + lane]), vv1 = bf2f(pool[kb + voff + lane]);
      const float sc = wave_sum(qv * kv);  // raw score, as m (scaled in the exponent)
      const float m_new = fmaxf(m, sc);
      const float alpha = __builtin_amdgcn_exp2f((m - m_new) * c2);  // m = -inf: 0
      const float p = __builtin_amdgcn_exp2f((sc - m_new) * c2);
      l = l * alpha + p;
      acc = acc * alpha + p * vv1;
      m = m_new;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    reinterpret_cast<bf16_t*>(a.out)[(int64_t)i * d + head * HD + lane] = (bf16_t)f2bf(acc * inv);
  }
}

}  // namespace

namespace allie {

hipError_t launch_extend_prepare(const ExtendPrepArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(extend_prepare_kernel, dim3(1), dim3(PREP_THREADS), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_extend_tiles(const int32_t* group_start, int first_group, int n_groups, int32_t* tiles,
                               hipStream_t st) {
  if (first_group >= n_groups) return hipSuccess;
  hipLaunchKernelGGL(extend_tiles_kernel, dim3(1), dim3(PREP_THREADS), 0, st, group_start, first_group, n_groups,
                     tiles);
  return hipGetLastError();
}

hipError_t launch_attn_extend_wave(const ExtendAttnArgs& a, hipStream_t st) {
  const int64_t waves = (int64_t)a.n * a.n_head;
  if (waves == 0) return hipSuccess;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (a.act_bf16)
    hipLaunchKernelGGL(attn_extend_wave_kernel<bf16_t>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(attn_extend_wave_kernel<float>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_attn_extend_fan(const ExtendAttnArgs& a, int g0, hipStream_t st) {
  if (!a.act_bf16) return hipErrorInvalidValue;
  const int W = fan_waves(a.max_blocks);
  const size_t lds = (size_t)W * (FAN_TILE * 2 + 64 * 4);
  if (a.n_groups > g0)
    hipLaunchKernelGGL(attn_extend_fan_kernel, dim3(a.n_groups - g0, a.n_head), dim3(64 * W), lds, st, a, g0);
  return hipGetLastError();
}

hipError_t launch_attn_extend_tree(const ExtendAttnArgs& a, hipStream_t st) {
  if (!a.act_bf16 || a.tiles == nullptr) return hipErrorInvalidValue;
  if (a.n_tiles == 0) return hipSuccess;
  hipLaunchKernelGGL(attn_extend_tree_kernel, dim3(a.n_tiles, a.n_head), dim3(128), 0, st, a);
  return hipGetLastError();
}

}  // namespace allie
