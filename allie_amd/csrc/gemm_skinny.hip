// Skinny GEMMs (M <= 8 rows): C[m][n] = epi(sum_k A[m][k] W[n][k]).
//
// One new token per MCTS leaf (or a handful of leaves) makes every
// projection a matrix-vector product: the cost is streaming the weights
// (2 B per weight, 25 MB per layer of the medium model), and an MFMA tile
// kernel at M = 1 keeps only N / 128 workgroups busy and needs a K-split
// reduction pass.  Here a workgroup owns 4 output columns and walks K in
// 16-byte chunks per lane, so each weight byte is read once; the <= 8
// activation rows come from L2.  Narrow outputs (N < 2048: the attention and
// MLP output projections) use 4 waves per workgroup that take every 4th
// chunk, so N / 4 workgroups still occupy every SIMD; wider ones use one
// wave.  Sums are fp32 (VALU FMAs, no MFMA: at M <= 8 the work is at most 2
// FLOP per weight byte read; above that the MFMA kernels are faster).  The
// 4 x MR per-lane partial sums are reduced across the wave by halving
// exchanges (each step swaps the half a lane does not keep with its
// partner), the waves' results are added through LDS, and the epilogue of
// the MFMA kernels is applied element-wise:
//   EPI_STORE  C = bf16(acc + b)     EPI_GELU  C = bf16(gelu(bf16(acc + b)))
//   EPI_RESID  R += bf16(acc + b)    out_f32   C = acc + b
// with fp8 weights scaled per output channel before the bias.
//
// At these sizes a kernel costs its launch and one round trip to HBM, a few
// microseconds, whatever its bytes.  So the LayerNorm before a projection
// (ln_1 before QKV, ln_2 before c_fc, ln_f before the heads) runs in the
// projection's prologue instead of a kernel of its own: each workgroup first
// requests its weights, then normalises the <= 8 rows (a few KiB read from
// L2) into LDS while they arrive.  And the QKV projection of an extend
// writes its keys and values to their pool slots itself.
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int SK_COLS = 4;  // output columns per workgroup

constexpr int LN_MAX_NV = SKINNY_LN_MAX_K / 256;  // float4 groups per lane of a LayerNorm row

// 8 consecutive weights as stored (bf16: 16 bytes, fp8: 8 bytes)
template <int WT>
struct W8 {
  uint4 v;
};
template <>
struct W8<W_FP8> {
  uint2 v;
};
template <int WT>
ALLIE_DEV void fetch_w8(const void* W, int64_t off, W8<WT>& r) {
  if constexpr (WT == W_FP8)
    r.v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(W) + off);
  else
    r.v = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(W) + off);
}
template <int WT>
ALLIE_DEV void widen_w8(const W8<WT>& r, float (&w)[8]) {
  if constexpr (WT == W_FP8) {
    const uint32_t b[2] = {r.v.x, r.v.y};
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) w[4 * j + e] = fp8e4m3_to_f32((b[j] >> (8 * e)) & 0xffu);
  } else {
    const uint32_t b[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[2 * j] = __uint_as_float(b[j] << 16);
      w[2 * j + 1] = __uint_as_float(b[j] & 0xffff0000u);
    }
  }
}

// A[m][0 .. K) = bf16(LayerNorm(row m of a.ln_h)) into LDS, one wave per
// row.  Lane layout (lane owns float4 groups i * 64 + lane) and expressions
// are those of the LayerNorm kernel (norm.hip); gamma and beta load with the
// row, and the two sums over the wave run in registers (wave_sum_regs), so a
// statistic can differ from that kernel's in its last bit.
template <int WPB>
ALLIE_DEV void ln_prologue(const GemmArgs& a, bf16_t* __restrict__ sA) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K, nv = K >> 8;
  for (int m = wave; m < a.M; m += WPB) {
    const int64_t src = a.ln_row ? (int64_t)a.ln_row[m] : m;
    const float* __restrict__ hr = a.ln_h + src * K;
    float4 v[LN_MAX_NV], gg[LN_MAX_NV], bb[LN_MAX_NV];
#pragma unroll
    for (int i = 0; i < LN_MAX_NV; ++i) {
      if (i < nv) {
        const int c = (i * 64 + lane) * 4;
        v[i] = *reinterpret_cast<const float4*>(hr + c);
        gg[i] = *reinterpret_cast<const float4*>(a.ln_g + c);
        bb[i] = *reinterpret_cast<const float4*>(a.ln_b + c);
      }
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < LN_MAX_NV; ++i)
      if (i < nv) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float mean = wave_sum_regs(s) / (float)K;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < LN_MAX_NV; ++i) {
      if (i < nv) {
        float p0 = v[i].x - mean, p1 = v[i].y - mean, p2 = v[i].z - mean, p3 = v[i].w - mean;
        q += (p0 * p0 + p1 * p1) + (p2 * p2 + p3 * p3);
      }
    }
    const float rstd = rsqrtf(wave_sum_regs(q) / (float)K + a.ln_eps);
#pragma unroll
    for (int i = 0; i < LN_MAX_NV; ++i) {
      if (i < nv) {
        const int c = (i * 64 + lane) * 4;
        const float o0 = (v[i].x - mean) * rstd * gg[i].x + bb[i].x;
        const float o1 = (v[i].y - mean) * rstd * gg[i].y + bb[i].y;
        const float o2 = (v[i].z - mean) * rstd * gg[i].z + bb[i].z;
        const float o3 = (v[i].w - mean) * rstd * gg[i].w + bb[i].w;
        *reinterpret_cast<uint2*>(sA + (int64_t)m * K + c) = make_uint2(pack_bf16x2(o0, o1), pack_bf16x2(o2, o3));
      }
    }
  }
  __syncthreads();
}

// LNP: A is the LayerNorm of a.ln_h's rows, computed into LDS (dynamic
// shared memory of MR * K bf16) after the first two k-steps' weights were
// requested
template <int EPI, int WT, bool F32OUT, int MR, int WPB, bool LNP>
__global__ __launch_bounds__(64 * WPB) void gemm_skinny_kernel(GemmArgs a) {
  constexpr int NV = SK_COLS * MR;  // partial sums per lane: index c * MR + m
  extern __shared__ __align__(16) bf16_t sk_a[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * SK_COLS;
  const int M = a.M, K = a.K;
  const int k0 = (wave * 64 + lane) * 8;
  constexpr int KSTEP = 512 * WPB;
  W8<WT> pre[2][SK_COLS];
  if constexpr (LNP) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
      if (k0 + p * KSTEP < K)
#pragma unroll
        for (int c = 0; c < SK_COLS; ++c) fetch_w8<WT>(a.W, (int64_t)(n0 + c) * K + k0 + p * KSTEP, pre[p][c]);
    ln_prologue<WPB>(a, sk_a);
  }
  // the output this lane writes after the reductions (see below): value
  // base = c * MR + m of the lanes with (lane & (OMIN - 1)) == 0 (of wave 0
  // when WPB > 1); its bias, fp8 scale and residual load now, so the
  // epilogue waits on no memory
  constexpr int OMIN = 64 / NV;  // the last halving offset
  int base = 0;
#pragma unroll
  for (int o = 32, half = NV / 2; o >= OMIN; o >>= 1, half >>= 1) base += (lane & o) ? half : 0;
  const int c_out = base / MR, m_out = base % MR, n_out = n0 + c_out;
  const bool writer = (lane & (OMIN - 1)) == 0 && m_out < M && (WPB == 1 || wave == 0);
  float bias_v = 0.f, scale_v = 1.f, r_v = 0.f;
  if (writer) {
    if (a.bias) bias_v = a.bias[n_out];
    if constexpr (WT == W_FP8) scale_v = a.scale[n_out];
    if constexpr (EPI == EPI_RESID && !F32OUT) r_v = a.R[(int64_t)m_out * a.ldr + n_out];
  }
  const bf16_t* A = reinterpret_cast<const bf16_t*>(a.A);
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = 0.f;
  int step = 0;
#pragma unroll 2
  for (int k = k0; k < K; k += KSTEP, ++step) {
    float w[SK_COLS][8];
    if (LNP && step < 2) {
#pragma unroll
      for (int c = 0; c < SK_COLS; ++c) widen_w8<WT>(step == 0 ? pre[0][c] : pre[1][c], w[c]);
    } else {
#pragma unroll
      for (int c = 0; c < SK_COLS; ++c) {
        W8<WT> r;
        fetch_w8<WT>(a.W, (int64_t)(n0 + c) * K + k, r);
        widen_w8<WT>(r, w[c]);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const uint4 x4 = LNP ? *reinterpret_cast<const uint4*>(sk_a + m * K + k)
                             : *reinterpret_cast<const uint4*>(A + (int64_t)m * a.lda + k);
        const uint32_t xb[4] = {x4.x, x4.y, x4.z, x4.w};
        float x[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[2 * j] = __uint_as_float(xb[j] << 16);
          x[2 * j + 1] = __uint_as_float(xb[j] & 0xffff0000u);
        }
#pragma unroll
        for (int c = 0; c < SK_COLS; ++c) {
          float s = v[c * MR + m];
#pragma unroll
          for (int j = 0; j < 8; ++j) s = fmaf(w[c][j], x[j], s);
          v[c * MR + m] = s;
        }
      }
    }
  }
  // reduce-scatter across the wave: at offset o a lane keeps the upper half
  // of its values if (lane & o), the lower half otherwise, and adds the
  // partner's copy of that half
#pragma unroll
  for (int o = 32, half = NV / 2; o >= OMIN; o >>= 1, half >>= 1) {
    const bool up = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float keep = up ? v[i + half] : v[i];
      const float send = up ? v[i] : v[i + half];
      v[i] = keep + __shfl_xor(send, o, 64);
    }
  }
  float r = v[0];
#pragma unroll
  for (int o = OMIN / 2; o > 0; o >>= 1) r += __shfl_xor(r, o, 64);
  if constexpr (WPB > 1) {
    __shared__ float part[WPB][NV];
    if ((lane & (OMIN - 1)) == 0) part[wave][base] = r;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < WPB; ++w) r += part[w][base];
  }
  if (!writer) return;
  const int m = m_out, n = n_out;
  if constexpr (WT == W_FP8) r *= scale_v;
  if (a.bias) r += bias_v;
  if constexpr (F32OUT) {
    reinterpret_cast<float*>(a.C)[(int64_t)m * a.ldc + n] = r;
  } else if constexpr (EPI == EPI_RESID) {
    a.R[(int64_t)m * a.ldr + n] = r_v + round_bf16(r);
  } else {
    if constexpr (EPI == EPI_GELU) r = gelu_tanh_fast(round_bf16(r));
    const bf16_t y = (bf16_t)f2bf(r);
    reinterpret_cast<bf16_t*>(a.C)[(int64_t)m * a.ldc + n] = y;
    if constexpr (EPI == EPI_STORE) {
      // an extend's QKV projection: keys and values also to their pool slot
      const int dm = a.N / 3;
      if (a.kv_pool && n >= dm) {
        const int sl = a.kv_slot[m];
        if (sl >= 0 && (sl >> 4) < a.kv_pool_blocks) {
          const int e = n - dm, kv = e >= dm ? 1 : 0, rem = e - kv * dm;
          const int64_t dst =
              (((((int64_t)a.kv_layer * a.kv_pool_blocks + (sl >> 4)) * 2 + kv) * (dm >> 6) + (rem >> 6)) * KV_BLOCK +
               (sl & 15)) * 64 + (rem & 63);
          reinterpret_cast<bf16_t*>(a.kv_pool)[dst] = y;
        }
      }
    }
  }
}

template <int EPI, int WT, bool F32OUT, int WPB, bool LNP>
void launch_rows_ln(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.N / SK_COLS)), block(64 * WPB);
  const uint32_t lds = LNP ? (uint32_t)(a.M <= 1 ? 1 : (a.M <= 4 ? 4 : 8)) * a.K * 2 : 0;
  if (a.M <= 1)
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 1, WPB, LNP>, grid, block, lds, st, a);
  else if (a.M <= 4)
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 4, WPB, LNP>, grid, block, lds, st, a);
  else
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 8, WPB, LNP>, grid, block, lds, st, a);
}

template <int EPI, int WT, bool F32OUT, int WPB>
void launch_rows(const GemmArgs& a, hipStream_t st) {
  // the LayerNorm prologue feeds only the projections that follow a
  // LayerNorm (no residual epilogue)
  if constexpr (EPI != EPI_RESID) {
    if (a.ln_h) return launch_rows_ln<EPI, WT, F32OUT, WPB, true>(a, st);
  }
  launch_rows_ln<EPI, WT, F32OUT, WPB, false>(a, st);
}

template <int EPI, int WT, bool F32OUT>
hipError_t launch_cols(const GemmArgs& a, hipStream_t st) {
  if (a.N < 2048)
    launch_rows<EPI, WT, F32OUT, 4>(a, st);
  else
    launch_rows<EPI, WT, F32OUT, 1>(a, st);
  return hipGetLastError();
}

template <int WT>
hipError_t launch_wt(const GemmArgs& a, hipStream_t st) {
  if (a.out_f32) return a.epi == EPI_STORE ? launch_cols<EPI_STORE, WT, true>(a, st) : hipErrorInvalidValue;
  switch (a.epi) {
    case EPI_STORE: return launch_cols<EPI_STORE, WT, false>(a, st);
    case EPI_GELU: return launch_cols<EPI_GELU, WT, false>(a, st);
    case EPI_RESID: return launch_cols<EPI_RESID, WT, false>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

namespace allie {

bool gemm_skinny_ln_ok(int M, int N, int K, int wtype) {
  return M >= 1 && M <= SKINNY_MAX_M && (wtype == W_BF16 || wtype == W_FP8) && N % SK_COLS == 0 && K % 256 == 0 &&
         K <= SKINNY_LN_MAX_K;
}

bool gemm_skinny_supported(const GemmArgs& a) {
  if (a.M < 1 || a.M > SKINNY_MAX_M) return false;
  if (a.wtype != W_BF16 && a.wtype != W_FP8) return false;
  if (a.wtype == W_FP8 && a.scale == nullptr) return false;
  if (a.N % SK_COLS != 0 || a.K % 8 != 0 || a.lda % 8 != 0) return false;
  if (a.out_f32 && a.epi != EPI_STORE) return false;
  if (a.epi == EPI_RESID && a.R == nullptr) return false;
  if (a.ln_h) {
    if (!gemm_skinny_ln_ok(a.M, a.N, a.K, a.wtype) || a.epi == EPI_RESID || !a.ln_g || !a.ln_b) return false;
    return (reinterpret_cast<uintptr_t>(a.W) & 15) == 0;
  }
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W);
  return (al & 15) == 0;
}

hipError_t launch_gemm_skinny(const GemmArgs& a, hipStream_t st) {
  if (!gemm_skinny_supported(a)) return hipErrorInvalidValue;
  return a.wtype == W_FP8 ? launch_wt<W_FP8>(a, st) : launch_wt<W_BF16>(a, st);
}

}  // namespace allie
