// Attention kernels.
//
// The reference runs GPT-2 attention through torch SDPA via BetterTransformer
// (src/modeling/model.py:190): per head softmax(q k^T / sqrt(hd)) v with a
// causal mask, plus key padding at B > 1.  On a packed ragged stream the
// padding disappears: query i of a game sees keys 0..i of the same game.
//
// attn_varlen_bf16_kernel -- one workgroup per (query tile of 64 rows, head),
// two waves of 32 query rows, key/value tiles of 64 through LDS.  Scores are
// computed transposed, S^T = K Q^T, with MFMA 32x32x16 bf16, so every lane
// owns one query (column l % 32) and 16 of the 32 keys of a block: the row
// max and row sum need one exchange with lane l ^ 32 only.  The output is
// likewise accumulated transposed, O^T = V^T P^T: P^T is already in the
// B-operand layout lane by lane (after a fixed permutation of the key index
// that is applied identically to V^T), and V^T comes from a transposed,
// padded LDS copy of the value tile.  Online softmax in fp32 with exp2; P
// enters the PV product as two bf16 MFMA operands, hi = bf16(p) and
// lo = bf16(p - hi), so the weights keep ~16 mantissa bits (a single bf16 P
// costs up to 2^-9 relative per weight, enough to flip the bf16 rounding of
// many attention outputs against an fp32-softmax reference).
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int QT = ATTN_Q_TILE;  // 64 query rows per workgroup
constexpr int KT = 64;           // keys per LDS tile
constexpr int HD = 64;           // head dim (GPT-2: d_model / n_head = 64)
constexpr int VT_LD = KT + 4;    // padded row of the transposed value tile
constexpr int MAX_KEYS_F32 = 512;  // fp32 kernel: keys per query held in LDS

ALLIE_DEV int kswz(int row, int chunk) { return row * HD + ((chunk ^ (row & 7)) << 3); }

__global__ __launch_bounds__(128) void attn_varlen_bf16_kernel(AttnVarlenArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t sK[KT * HD];
  __shared__ __attribute__((aligned(16))) bf16_t sVt[HD * VT_LD];

  const int head = blockIdx.x;
  const int tile = a.tiles[blockIdx.y];
  const int s = tile >> 5, qt = tile & 31;
  const int t0 = a.cu_seqlens[s];
  const int n = a.cu_seqlens[s + 1] - t0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, ql = lane & 31;
  const int d = a.n_head * HD;
  const int ld = 3 * d;
  const bf16_t* __restrict__ qkv = reinterpret_cast<const bf16_t*>(a.qkv);

  // Q fragment (B operand of S^T = K Q^T): query q_pos, hd 16 kk + 8 g .. +7
  const int q_pos = qt * QT + wave * 32 + ql;
  bf16x8_t qf[4];
  {
    const bool ok = q_pos < n;
    const bf16_t* qrow = qkv + (int64_t)(t0 + (ok ? q_pos : 0)) * ld + head * HD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4_t v = ok ? *reinterpret_cast<const u32x4_t*>(qrow + kk * 16 + g * 8) : u32x4_t{0, 0, 0, 0};
      qf[kk] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  const float sl2 = a.scale * 1.4426950408889634f;  // scale * log2(e)
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};

  const int kv_end = min(n, (qt + 1) * QT);  // keys visible to this tile
  for (int k0 = 0; k0 < kv_end; k0 += KT) {
    // ---- stage K (swizzled rows) and V^T (padded) -----------------------
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cidx = tid + 128 * i;  // 512 chunks: 64 keys x 8 chunks
      const int key = cidx >> 3, c = cidx & 7;
      const bool ok = k0 + key < n;
      const bf16_t* row = qkv + (int64_t)(t0 + k0 + key) * ld + head * HD + c * 8;
      uint4 kv = ok ? *reinterpret_cast<const uint4*>(row + d) : make_uint4(0, 0, 0, 0);
      uint4 vv = ok ? *reinterpret_cast<const uint4*>(row + 2 * d) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&sK[kswz(key, c)]) = kv;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sVt[(c * 8 + 2 * j) * VT_LD + key] = (bf16_t)(w[j] & 0xffffu);
        sVt[(c * 8 + 2 * j + 1) * VT_LD + key] = (bf16_t)(w[j] >> 16);
      }
    }
    __syncthreads();

    // ---- S^T for two 32-key blocks ----------------------------------------
    f32x16_t st[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      st[b] = f32x16_t{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int krow = b * 32 + ql;
        bf16x8_t kf = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sK[kswz(krow, kk * 2 + g)]));
        st[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], st[b], 0, 0, 0);
      }
    }
    // ---- mask + online softmax (lane owns query q_pos) -------------------
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + b * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        float v = st[b][r] * sl2;
        if (key > q_pos || key >= n) v = -INFINITY;
        st[b][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);  // m_run = -inf first: alpha = 0
    m_run = m_new;
    float ls = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(st[b][r] - m_new);
        st[b][r] = p;
        ls += p;
      }
    l_run = l_run * alpha + ls;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[hb][r] *= alpha;

    // ---- O^T += V^T P^T --------------------------------------------------
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        // P = P_hi + P_lo, both bf16: the PV product keeps ~16 mantissa bits of
        // the fp32 probabilities instead of bf16's 8
        bf16x8_t pf, pl;
        if (mm == 0) split_bf16x8<0>(st[b], pf, pl); else split_bf16x8<8>(st[b], pf, pl);
        const int kb = b * 32 + mm * 16 + 4 * g;  // keys kb..kb+3 and kb+8..kb+11
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const bf16_t* vr = &sVt[(hb * 32 + ql) * VT_LD];
          u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr + kb);
          u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + kb + 8);
          bf16x8_t vf = __builtin_bit_cast(bf16x8_t, u32x4_t{lo.x, lo.y, hi.x, hi.y});
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[hb], 0, 0, 0);
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pl, o[hb], 0, 0, 0);
        }
      }
  }
  // ---- normalise and store: lane holds hd 8 (r/4) + 4 g + r%4 of q_pos ----
  if (q_pos >= n) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l_tot;
  bf16_t* out = reinterpret_cast<bf16_t*>(a.out) + (int64_t)(t0 + q_pos) * d + head * HD;
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int hd = hb * 32 + q4 * 8 + 4 * g;
      uint2 p;
      p.x = pack_bf16x2(o[hb][q4 * 4 + 0] * inv, o[hb][q4 * 4 + 1] * inv);
      p.y = pack_bf16x2(o[hb][q4 * 4 + 2] * inv, o[hb][q4 * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(out + hd) = p;
    }
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
    const int64_t dst = ((((blk * a.n_layer + a.layer) * 2 + kvi) * H + head) * KV_BLOCK + off) * hd + i;
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
    if (a.n_tiles == 0) return hipSuccess;
    if (a.n_tiles > 65535) return hipErrorInvalidValue;  // grid y limit
    hipLaunchKernelGGL(attn_varlen_bf16_kernel, dim3(a.n_head, a.n_tiles), dim3(128), 0, st, a);
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
