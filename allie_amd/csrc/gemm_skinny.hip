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
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int SK_COLS = 4;  // output columns per workgroup

template <int WT>
ALLIE_DEV void load_w8(const void* W, int64_t off, float (&w)[8]) {
  if constexpr (WT == W_FP8) {
    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(W) + off);
    const uint32_t b[2] = {v.x, v.y};
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) w[4 * j + e] = fp8e4m3_to_f32((b[j] >> (8 * e)) & 0xffu);
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(W) + off);
    const uint32_t b[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[2 * j] = __uint_as_float(b[j] << 16);
      w[2 * j + 1] = __uint_as_float(b[j] & 0xffff0000u);
    }
  }
}

template <int EPI, int WT, bool F32OUT, int MR, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemm_skinny_kernel(GemmArgs a) {
  constexpr int NV = SK_COLS * MR;  // partial sums per lane: index c * MR + m
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * SK_COLS;
  const int M = a.M, K = a.K;
  const bf16_t* A = reinterpret_cast<const bf16_t*>(a.A);
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = 0.f;
#pragma unroll 2
  for (int k = (wave * 64 + lane) * 8; k < K; k += 512 * WPB) {
    float w[SK_COLS][8];
#pragma unroll
    for (int c = 0; c < SK_COLS; ++c) load_w8<WT>(a.W, (int64_t)(n0 + c) * K + k, w[c]);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const uint4 x4 = *reinterpret_cast<const uint4*>(A + (int64_t)m * a.lda + k);
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
  int base = 0;
  constexpr int OMIN = 64 / NV;  // the last halving offset
#pragma unroll
  for (int o = 32, half = NV / 2; o >= OMIN; o >>= 1, half >>= 1) {
    const bool up = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float keep = up ? v[i + half] : v[i];
      const float send = up ? v[i] : v[i + half];
      v[i] = keep + __shfl_xor(send, o, 64);
    }
    base += up ? half : 0;
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
  if ((lane & (OMIN - 1)) != 0) return;
  const int c = base / MR, m = base % MR;
  if (m >= M) return;
  const int n = n0 + c;
  if constexpr (WT == W_FP8) r *= a.scale[n];
  if (a.bias) r += a.bias[n];
  if constexpr (F32OUT) {
    reinterpret_cast<float*>(a.C)[(int64_t)m * a.ldc + n] = r;
  } else if constexpr (EPI == EPI_RESID) {
    a.R[(int64_t)m * a.ldr + n] += round_bf16(r);
  } else {
    if constexpr (EPI == EPI_GELU) r = gelu_tanh_fast(round_bf16(r));
    reinterpret_cast<bf16_t*>(a.C)[(int64_t)m * a.ldc + n] = (bf16_t)f2bf(r);
  }
}

template <int EPI, int WT, bool F32OUT, int WPB>
void launch_rows(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.N / SK_COLS)), block(64 * WPB);
  if (a.M <= 1)
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 1, WPB>, grid, block, 0, st, a);
  else if (a.M <= 4)
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 4, WPB>, grid, block, 0, st, a);
  else
    launch_timed(gemm_skinny_kernel<EPI, WT, F32OUT, 8, WPB>, grid, block, 0, st, a);
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

bool gemm_skinny_supported(const GemmArgs& a) {
  if (a.M < 1 || a.M > SKINNY_MAX_M) return false;
  if (a.wtype != W_BF16 && a.wtype != W_FP8) return false;
  if (a.wtype == W_FP8 && a.scale == nullptr) return false;
  if (a.N % SK_COLS != 0 || a.K % 8 != 0 || a.lda % 8 != 0) return false;
  if (a.out_f32 && a.epi != EPI_STORE) return false;
  if (a.epi == EPI_RESID && a.R == nullptr) return false;
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W);
  return (al & 15) == 0;
}

hipError_t launch_gemm_skinny(const GemmArgs& a, hipStream_t st) {
  if (!gemm_skinny_supported(a)) return hipErrorInvalidValue;
  return a.wtype == W_FP8 ? launch_wt<W_FP8>(a, st) : launch_wt<W_BF16>(a, st);
}

}  // namespace allie
