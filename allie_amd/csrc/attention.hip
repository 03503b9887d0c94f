// Attention kernels.
//
// The reference runs GPT-2 attention through torch SDPA via BetterTransformer
// (src/modeling/model.py:190): per head softmax(q k^T / sqrt(hd)) v with a
// causal mask, plus key padding at B > 1.  On a packed ragged stream the
// padding disappears: query i of a game sees keys 0..i of the same game.
//
// attn_varlen_seq_kernel -- one workgroup of 8 waves per (game, 4 heads), or per
// (game, head) when there are fewer than 64 games.
// A head's keys and values (bf16) of the whole game are staged in LDS (at
// most 512 tokens, 128 KiB); each wave then takes 32-query tiles in an order
// that balances the causal work (tile t costs t + 1 key blocks) and waits
// for the others only when the next head (loaded into registers meanwhile)
// is staged.  Per 32-key block: S^T = K Q^T with MFMA 32x32x16 bf16, so a
// lane owns one query and 16 keys (the row max and sum need one exchange
// with lane l ^ 32); online softmax in fp32 with exp2, the accumulator
// rescaled only when some lane's running max grows.  As in torch's bf16
// SDPA kernels, P = exp(s - max) enters the PV product rounded to bf16
// (nearest even) while the row sum adds the unrounded fp32 P; O^T += V^T P^T
// runs on MFMA 32x32x16 bf16, whose V^T fragments come straight from the
// row-major value rows through gfx950's transposing LDS read
// (ds_read_b64_tr_b16).
//
// Grid: (head group, game), the games in order of decreasing length
// (seq_order_kernel, a counting sort) so that the longest start first.
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int HD = 64;           // head dim (GPT-2: d_model / n_head = 64)
constexpr int MAX_KEYS_F32 = 512;  // fp32 kernel: keys per query held in LDS
constexpr int SEQ_WAVES = 8;       // waves per workgroup of the per-game kernel
constexpr int SEQ_MAXN = 512;      // longest game it stages (max_length)
constexpr int SEQ_HEADS = 4;       // heads per workgroup (the next one loads during one), B >= SEQ_FEW
constexpr int SEQ_FEW = 64;        // fewer games: one head per workgroup, so a batch of one
                                   // game still spreads over n_head workgroups

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

__global__ __launch_bounds__(SEQ_WAVES * 64, 1) void attn_varlen_seq_kernel(AttnVarlenArgs a) {
  // K rows: 128 B, 16-byte chunk c of row r at c ^ ((r >> 1) & 7) (16
  // consecutive rows reading one chunk hit distinct bank groups).  V rows:
  // 128 B, 8-byte chunk j of row r at j ^ (4 ((r >> 1) & 1)) (the 4 x 16
  // blocks the transposing read takes hit distinct bank groups).
  __shared__ __attribute__((aligned(1024))) uint16_t sK[SEQ_MAXN * HD];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[SEQ_MAXN * HD];

  const int s = a.order[blockIdx.y];
  const int t0 = a.cu_seqlens[s];
  int n = a.cu_seqlens[s + 1] - t0;
  if (n <= 0) return;
  n = n < SEQ_MAXN ? n : SEQ_MAXN;
  const int npad = (n + 31) & ~31;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = a.n_head * HD, ld = 3 * d;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);

  // ---- staging of one head's keys and values (rows past n are zero): the
  // loads of the next head are in flight while this one is computed --------
  constexpr int PER = SEQ_MAXN * 8 / (SEQ_WAVES * 64);  // 16-byte chunks per thread
  uint4 kv[PER], vv[PER];
  auto load_head = [&](int head) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * SEQ_WAVES * 64;
      const int row = c >> 3, ch = c & 7;
      kv[i] = make_uint4(0, 0, 0, 0);
      vv[i] = make_uint4(0, 0, 0, 0);
      if (row < n) {
        const bf16_t* src = qkv + (int64_t)(t0 + row) * ld + head * HD + ch * 8;
        kv[i] = *reinterpret_cast<const uint4*>(src + d);
        vv[i] = *reinterpret_cast<const uint4*>(src + 2 * d);
      }
    }
  };
  auto store_head = [&]() {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * SEQ_WAVES * 64;
      const int row = c >> 3, ch = c & 7;
      if (row >= npad) break;
      *reinterpret_cast<uint4*>(sK + row * HD + ((ch ^ ((row >> 1) & 7)) << 3)) = kv[i];
      // 16 bytes = 8-byte chunks 2 ch, 2 ch + 1: the swizzle moves them together
      *reinterpret_cast<uint4*>(sV + row * HD + ((ch ^ (((row >> 1) & 1) << 1)) << 3)) = vv[i];
    }
  };
  const int hpw = (a.n_head + gridDim.x - 1) / gridDim.x;  // heads per workgroup (grid x = head groups)
  const int h_first = blockIdx.x * hpw;
  const int h_end = h_first + hpw < a.n_head ? h_first + hpw : a.n_head;
  load_head(h_first);
  store_head();
  __syncthreads();

  const int ql = lane & 31, g = lane >> 5;
  const float c2 = a.scale * 1.4426950408889634f;  // scale * log2(e)
  // transposing V read of lane l: row (l % 16) / 4 of a 4-key group, dims
  // hd0 + 4 (l % 4) .. + 3 with hd0 = 16 ((l / 16) % 2)
  const int trow = (lane & 15) >> 2;
  const int tchunk = ((lane >> 4) & 1) * 4 + (lane & 3);  // 8-byte chunk inside a 32-dim block
  bf16_t* __restrict__ out = reinterpret_cast<bf16_t*>(a.out);

  auto tile = [&](int head, int qt) {
    const int q0 = qt * 32;
    const int qrow = q0 + ql < n ? q0 + ql : n - 1;
    bf16x8_t qf[4];
    {
      const bf16_t* qp = qkv + (int64_t)(t0 + qrow) * ld + head * HD + g * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(qp + kk * 16));
    }
    float m = -INFINITY, lsum = 0.f;
    f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};
    auto load_k = [&](int kb, bf16x8_t (&kf)[4]) {
      const int krow = kb * 32 + ql;
      const uint16_t* kr = sK + krow * HD;
      const int sw = (krow >> 1) & 7;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        kf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(kr + (((2 * kk + g) ^ sw) << 3)));
    };
    // a block's key fragments are read while the previous block is scored
    bf16x8_t kf[4];
    load_k(0, kf);
    for (int kb = 0; kb <= qt; ++kb) {
      f32x16_t st{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[kk], st, 0, 0, 0);
      load_k(kb < qt ? kb + 1 : kb, kf);  // (the last block re-reads its own, in bounds)
      // lane holds keys 8 (r / 4) + 4 g + r % 4 of the block for query ql
      if (kb == qt) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (8 * (r >> 2) + 4 * g + (r & 3) > ql) st[r] = -INFINITY;
      }
      float mx = st[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, st[r]);
      mx = xor32_max(mx);
      const float m_new = fmaxf(m, mx);
      if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {
        const float alpha = __builtin_amdgcn_exp2f((m - m_new) * c2);  // m = -inf first: 0
        lsum *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o[0][r] *= alpha;
          o[1][r] *= alpha;
        }
      }
      m = m_new;
      const float mc = m_new * c2;
      uint32_t pk[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(st[r], c2, -mc));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(st[r + 1], c2, -mc));
        lsum += p0 + p1;
        pk[r >> 1] = pack_bf16x2(p0, p1);
      }
      // ---- O^T += V^T P^T: k-step mm covers keys 16 mm + {4 g .. 4 g + 3,
      // 8 + 4 g .. 8 + 4 g + 3} (the S^T layout), identically for V^T -----
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[4 * mm], pk[4 * mm + 1], pk[4 * mm + 2], pk[4 * mm + 3]});
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          bf16x4_t lo, hi;
          {
            const int r0 = kb * 32 + 16 * mm + 4 * g + trow;  // rows of the two 4-key groups
            const int r1 = r0 + 8;
            const int j = hb * 8 + tchunk;
            lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r0 * HD + ((j ^ (((r0 >> 1) & 1) << 2)) << 2)));
            hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                (lds_bf16x4_t*)((__attribute__((address_space(3))) uint16_t*)sV + r1 * HD + ((j ^ (((r1 >> 1) & 1) << 2)) << 2)));
          }
          const bf16x8_t vf = __builtin_bit_cast(
              bf16x8_t, u32x4_t{__builtin_bit_cast(u32x2_t, lo).x, __builtin_bit_cast(u32x2_t, lo).y,
                                __builtin_bit_cast(u32x2_t, hi).x, __builtin_bit_cast(u32x2_t, hi).y});
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[hb], 0, 0, 0);
        }
      }
    }
    // ---- normalise and store: lane holds dims 32 hb + 8 (r / 4) + 4 g + r % 4
    if (q0 + ql >= n) return;
    const float inv = 1.0f / xor32_sum(lsum);
    bf16_t* orow = out + (int64_t)(t0 + q0 + ql) * d + head * HD;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint2 pv;
        pv.x = pack_bf16x2(o[hb][q4 * 4 + 0] * inv, o[hb][q4 * 4 + 1] * inv);
        pv.y = pack_bf16x2(o[hb][q4 * 4 + 2] * inv, o[hb][q4 * 4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + hb * 32 + q4 * 8 + 4 * g) = pv;
      }
  };

  // per head: 32-query tiles, heaviest first, dealt to the waves in a snake
  // order; then every wave is done with the staged head and the next one
  // (loaded meanwhile) takes its place
  const int T32 = npad / 32;
  const int n_run = a.last_only ? 1 : T32;  // last_only: the tile holding the last query
  for (int head = h_first; head < h_end; ++head) {
    const bool more = head + 1 < h_end;
    if (more) load_head(head + 1);
    for (int r = 0; r * SEQ_WAVES < n_run; ++r) {
      const int idx = r * SEQ_WAVES + ((r & 1) ? SEQ_WAVES - 1 - wave : wave);
      if (idx < n_run) tile(head, T32 - 1 - idx);
    }
    if (!more) break;
    __syncthreads();
    store_head();
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Games by decreasing length (a counting sort over lengths 0 .. SEQ_MAXN,
// longer ones clamped; order within a length is arbitrary).  One workgroup.
constexpr int ORDER_THREADS = 1024;
__global__ __launch_bounds__(ORDER_THREADS) void seq_order_kernel(const int32_t* __restrict__ cu, int B,
                                                                  int32_t* __restrict__ order) {
  __shared__ int bin[SEQ_MAXN + 1];
  for (int i = threadIdx.x; i <= SEQ_MAXN; i += ORDER_THREADS) bin[i] = 0;
  __syncthreads();
  auto len_of = [&](int s) {
    int n = cu[s + 1] - cu[s];
    return n < 0 ? 0 : (n > SEQ_MAXN ? SEQ_MAXN : n);
  };
  for (int s = threadIdx.x; s < B; s += ORDER_THREADS) atomicAdd(&bin[len_of(s)], 1);
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive scan from the longest length down
    int acc = 0;
    for (int l = SEQ_MAXN; l >= 0; --l) {
      const int c = bin[l];
      bin[l] = acc;
      acc += c;
    }
  }
  __syncthreads();
  for (int s = threadIdx.x; s < B; s += ORDER_THREADS) order[atomicAdd(&bin[len_of(s)], 1)] = s;
}

// ---------------------------------------------------------------------------
// fp32 check-mode attention: one wave per (query token, head); lane j scores
// keys j, j + 64, ...; lane = head-dim index for the weighted sum.
__global__ __launch_bounds__(256) void attn_varlen_f32_kernel(AttnVarlenArgs a) {
  __shared__ float sp[4][MAX_KEYS_F32];
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int head = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool valid = t < a.T;
  int t0 = 0, i = -1;
  if (valid) {
    // binary search the game of token t: cu[lo] <= t < cu[lo + 1]
    int lo = 0, hi = a.B;
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (a.cu_seqlens[mid] <= t) lo = mid; else hi = mid;
    }
    t0 = a.cu_seqlens[lo];
    i = (int)(t - t0);
  }
  const int d = a.n_head * HD, ld = 3 * d;
  const float* __restrict__ qkv = reinterpret_cast<const float*>(a.qkv);
  const float* q = qkv + (valid ? t : 0) * ld + head * HD;
  float mx = -INFINITY;
  for (int j = lane; j <= i; j += 64) {
    const float* k = qkv + (int64_t)(t0 + j) * ld + d + head * HD;
    float s = 0.f;
#pragma unroll 8
    for (int c = 0; c < HD; ++c) s = fmaf(q[c], k[c], s);
    s *= a.scale;
    sp[w][j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = lane; j <= i; j += 64) {
    float p = __expf(sp[w][j] - mx);
    sp[w][j] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  __syncthreads();  // every thread reaches this: no early exit above
  if (!valid) return;
  float acc = 0.f;
  for (int j = 0; j <= i; ++j)
    acc = fmaf(sp[w][j], qkv[(int64_t)(t0 + j) * ld + 2 * d + head * HD + lane], acc);
  reinterpret_cast<float*>(a.out)[t * d + head * HD + lane] = acc / sum;
}


// ---------------------------------------------------------------------------
// KV cache write: token t's keys and values of one layer go to pool slot
// slot[t] (block slot/16, offset slot%16).  16 bytes per thread.
__global__ __launch_bounds__(256) void kv_write_kernel(KVWriteArgs a) {
  const int64_t t = blockIdx.x;
  const int H = a.n_head, hd = a.head_dim, d = H * hd;
  const int esz = a.act_bf16 ? 2 : 4;
  const int per_chunk = 16 / esz;                // elements per 16-byte chunk
  const int chunks = 2 * d / per_chunk;          // k and v of all heads
  const int sl = a.slot[t];
  if (sl < 0 || (sl >> 4) >= a.pool_blocks) return;  // flagged by the caller's validation
  const int64_t blk = sl >> 4, off = sl & 15;
  const char* src = reinterpret_cast<const char*>(a.qkv) + (t * 3 * d + d) * esz;  // k | v
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    const int e = c * per_chunk;                 // element in [0, 2d): kv * d + head * hd + i
    const int kvi = e / d, rem = e - kvi * d, head = rem / hd, i = rem - head * hd;
    const int64_t dst = (((((int64_t)a.layer * a.pool_blocks + blk) * 2 + kvi) * H + head) * KV_BLOCK + off) * hd + i;
    *reinterpret_cast<uint4*>(reinterpret_cast<char*>(a.pool) + dst * esz) =
        *reinterpret_cast<const uint4*>(src + (int64_t)e * esz);
  }
}

}  // namespace

namespace allie {

hipError_t launch_attn_varlen(const AttnVarlenArgs& a, hipStream_t st) {
  // callers guarantee every game has at most MAX_KEYS_F32 tokens (max_length)
  if (a.head_dim != HD) return hipErrorInvalidValue;
  if (a.act_bf16) {
    if (a.B <= 0) return hipSuccess;
    if (a.B > 65535 || !a.order) return hipErrorInvalidValue;  // grid y limit; workspace
    if (!a.order_ready)
      hipLaunchKernelGGL(seq_order_kernel, dim3(1), dim3(ORDER_THREADS), 0, st, a.cu_seqlens, a.B, a.order);
    const int hpw = a.B < SEQ_FEW ? 1 : SEQ_HEADS;
    launch_timed(attn_varlen_seq_kernel, dim3((a.n_head + hpw - 1) / hpw, a.B), dim3(SEQ_WAVES * 64), 0, st, a);
  } else {
    if (a.T == 0) return hipSuccess;
    hipLaunchKernelGGL(attn_varlen_f32_kernel, dim3((a.T + 3) / 4, a.n_head), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_kv_write(const KVWriteArgs& a, hipStream_t st) {
  if (a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_write_kernel, dim3(a.T), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace allie
