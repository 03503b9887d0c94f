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
// Groups of at most 16 tokens sharing a prefix (MCTS children of one node):
// one workgroup per (group, head) whose W waves take the prefix's 64-key
// chunks in turn (wave w: chunks w, w + W, ...), so a group's whole prefix
// is requested at once.  A wave holds all of the group's queries in 16x16x32
// MFMAs (S^T = K Q^T: key rows, query columns), loads its chunk's K
// fragments straight into MFMA registers (a lane's key row segment is
// contiguous), stages V as fp16 in its own LDS tile for the transposing
// read, and keeps its own running max / sum / O.  The waves' partials merge
// through LDS and wave w finishes tokens w, w + W, ... (lane = head dim):
// the private keys (ancestors, then the token itself) and the normalisation.
// Everything a wave needs for its first tokens' private keys is loaded
// before the prefix loop, so those loads overlap the prefix's.
constexpr int FAN_CHUNK = 64, FAN_TILE = FAN_CHUNK * HD;  // fp16 V tile (8 KiB); later the fp32 16 x 64 partial
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

// two bf16 (one word) -> two fp16 (exact for bf16 values in fp16's range)
ALLIE_DEV uint32_t bf16x2_to_f16x2(uint32_t w) { return pk_f16(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)); }

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
  const bf16_t* lbase = pool + ((int64_t)a.layer * 2 * H + head) * (KV_BLOCK * HD);
  const int64_t bstride = (int64_t)a.n_layer * 2 * H * KV_BLOCK * HD;
  auto slot_ok = [&](int sl) { return sl >= 0 && (sl >> 4) < a.pool_blocks; };
  auto slot_off = [&](int sl) { return pool_off(slot_ok(sl) ? sl >> 4 : 0, a.n_layer, a.layer, 0, H, head, sl & 15); };
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
        acc = acc * alpha + pe * bf2f(xv[t][e]);
        m = m_new;
      }
      xm[t] = m;
      xl[t] = l;
      xa[t] = acc;
    }
  };

  const int nch = (max(P, 0) + FAN_CHUNK - 1) / FAN_CHUNK;
  // pool block of (chunk c, block b); -1: skipped
  auto table_entry = [&](int c, int b) {
    const int bi = c * 4 + b;
    int v = -1;
    if (bi < a.max_blocks && bi * KV_BLOCK < P) v = btab[bi];
    return (v >= 0 && v < a.pool_blocks) ? v : -1;
  };
  // lane j holds block j % 4 of the wave's chunk j / 4 (its first 16 chunks)
  const int bt = table_entry(wave + W * (lane >> 2), lane & 3);
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
      blk[b] = __builtin_amdgcn_readfirstlane(n < 16 ? __builtin_amdgcn_readlane(bt, 4 * n + b) : table_entry(c, b));
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
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
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
        pf[s2] = u32x4_t{pk_f16(p[2 * s2][0], p[2 * s2][1]), pk_f16(p[2 * s2][2], p[2 * s2][3]),
                         pk_f16(p[2 * s2 + 1][0], p[2 * s2 + 1][1]), pk_f16(p[2 * s2 + 1][2], p[2 * s2 + 1][3])};
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    } else {
      pf[0] = pf[1] = u32x4_t{0, 0, 0, 0};
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the tile's DMA is done
    wave_lds_sync();
    // O^T += V^T P^T: A = V^T rows (dims 16 db + lq) in fp16, k-slots as
    // P^T's, read transposed: lane group lg reads keys 32 s + 4 lg + (lq >> 2)
    // (and + 16)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int r0 = 32 * s2 + 4 * lg + (lq >> 2), r1 = r0 + 16;
        const int j = 4 * db + (lq & 3);
        const fp16x4_ll lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r0 * HD + ((j ^ (((r0 >> 1) & 1) << 2)) << 2)));
        const fp16x4_ll hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (lds_f16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r1 * HD + ((j ^ (((r1 >> 1) & 1) << 2)) << 2)));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
        const u32x4_t vf{bf16x2_to_f16x2(l2.x), bf16x2_to_f16x2(l2.y), bf16x2_to_f16x2(h2.x), bf16x2_to_f16x2(h2.y)};
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, vf), __builtin_bit_cast(f16x8_t, pf[s2]),
                                                       o[db], 0, 0, 0);
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
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
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
        acc = acc * alpha + pe * bf2f(pool[kb + voff]);
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
  const size_t lds = (size_t)W * (FAN_TILE * 2 + 32 * 4);
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
