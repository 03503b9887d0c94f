// GEMMs of the transformer blocks and the heads on gfx950.
//
// C[m, n] = sum_k A[m, k] * W[n, k] with both operands K-contiguous: A is the
// activation stream [T][K] (bf16), W the weight matrix [N][K] (bf16, or fp8
// e4m3 with a per-output-channel fp32 scale).  This is the Conv1D
// ``addmm(b, x, W[in,out])`` of GPT-2 [lib transformers Conv1D] with the
// weights repacked once to [out][in] at load time.
//
// MFMA kernel: 256 threads (4 waves, 2 x 2), block tile 256 (M) x 256 (N),
// BK = 64, double-buffered LDS (2 x 64 KiB) filled by direct global->LDS
// 16-byte loads (fp8 weights go through registers to be widened to bf16),
// one block per CU.
// Each wave owns a 128 x 128 sub-tile = 4 x 4 MFMA 32x32x16 bf16 blocks
// (256 fp32 accumulators).  The MFMA's first operand is the weight fragment
// and its second the activation fragment, so each lane's accumulator holds 4
// consecutive output columns of one row: the epilogue stores 8 (bf16) or 16
// (fp32) contiguous bytes per lane.  LDS rows are 128 B (64 bf16); 16-byte
// chunk c of row r sits at chunk position c ^ (r & 7) so the fragment reads of
// 8 consecutive rows hit 8 distinct chunk positions.
//
// Block order: workgroups are dealt round-robin to the 8 XCDs, so block id
// pid runs on XCD pid % 8; tiles are renumbered so that each XCD walks a
// contiguous range of a grouped (GROUP_M m-tiles x all n-tiles) order and the
// tiles resident on one XCD share A rows and W rows in that XCD's L2.
//
// Epilogues (bf16 autocast semantics of the reference's addmm):
//   EPI_STORE  C = bf16(acc + b)               (QKV projection)
//   EPI_GELU   C = bf16(gelu(bf16(acc + b)))   (MLP c_fc + gelu_new)
//   EPI_RESID  R += bf16(acc + b)              (attn c_proj / MLP c_proj)
// with fp32 output (no rounding) when out_f32 is set (heads).
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NTHREADS = 256;
constexpr int GROUP_M = 4;

ALLIE_DEV int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 3); }

ALLIE_DEV void tile_coords(int pid, int G, int num_tm, int num_tn, int& tm, int& tn) {
  // XCD-aware renumbering: XCD x = pid % 8 takes a contiguous logical range
  const int xcd = pid & 7, idx = pid >> 3;
  const int per = G >> 3, rem = G & 7;
  const int logical = xcd * per + (xcd < rem ? xcd : rem) + idx;
  // grouped order: GROUP_M m-tiles x all n-tiles
  const int group_size = GROUP_M * num_tn;
  const int group = logical / group_size;
  const int first_m = group * GROUP_M;
  int gm = num_tm - first_m;
  gm = gm < GROUP_M ? gm : GROUP_M;
  const int in_group = logical - group * group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// fp8 weight tile (256 rows x 64 e4m3, register staged: 4 x 16 bytes per
// thread) -> bf16 into the swizzled LDS layout.
ALLIE_DEV void fp8_tile_to_lds(const uint4* rw, bf16_t* sw, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid >> 2) + 64 * i;
    const uint32_t w4[4] = {rw[i].x, rw[i].y, rw[i].z, rw[i].w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v = w4[j];
      o[2 * j] = fp8e4m3_to_bf16(v & 0xffu) | (fp8e4m3_to_bf16((v >> 8) & 0xffu) << 16);
      o[2 * j + 1] = fp8e4m3_to_bf16((v >> 16) & 0xffu) | (fp8e4m3_to_bf16(v >> 24) << 16);
    }
    const int c = (tid & 3) * 2;
    *reinterpret_cast<uint4*>(&sw[swz(row, c)]) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(&sw[swz(row, c + 1)]) = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Direct global -> LDS copy of 16 bytes per lane: the wave writes 1 KiB of
// LDS contiguously at `lds` (lane i at lds + 16 i).
ALLIE_DEV void g2l_16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 16, 0, 0);
}
ALLIE_DEV void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int EPI, int WT, bool OUT_F32>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_mfma_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) bf16_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(1024))) bf16_t sW[2][BN * BK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (LDS-DMA base)
  const int num_tm = (a.M + BM - 1) / BM, num_tn = a.N / BN;
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, num_tm, num_tn, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = a.K;
  const bf16_t* __restrict__ A = reinterpret_cast<const bf16_t*>(a.A);

  // Loader geometry: wave w fills rows [64 w, 64 w + 64) of each tile with 8
  // LDS-DMA instructions of 8 rows; lane -> (row 8 i + lane / 8, physical
  // chunk lane % 8), reading logical chunk (lane % 8) ^ (row & 7).
  const int lr = lane >> 3, pc = lane & 7, lcg = pc ^ lr;
  // rows of this lane: m0 + 64 wave + 8 i + lr (i = 0..7); rows at or past M
  // read the last valid row instead (their results are discarded)
  const int m_first = m0 + wave * 64 + lr;
  const int m_last_ok = a.M - 1 - m_first;  // copy i is in range iff 8 i <= m_last_ok
  const bf16_t* a_row0 = A + (int64_t)(m_first < a.M ? m_first : a.M - 1) * a.lda + lcg * 8;
  const bf16_t* a_last = A + (int64_t)(a.M - 1) * a.lda + lcg * 8;
  const int64_t a_step = (int64_t)8 * a.lda;
  const bf16_t* __restrict__ Wb = reinterpret_cast<const bf16_t*>(a.W);
  const bf16_t* w_row0 = Wb + (int64_t)(n0 + wave * 64 + lr) * K + lcg * 8;
  const int64_t w_step = (int64_t)8 * K;
  const uint8_t* __restrict__ W8 = reinterpret_cast<const uint8_t*>(a.W);
  uint4 rw[4];

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  const int wm = wave & 1, wn = wave >> 1;
  const int frow = lane & 31, fgrp = lane >> 5;
  const int KT = K / BK;

#define ISSUE_A(buf, k0)                                                              \
  _Pragma("unroll") for (int i = 0; i < 8; ++i) {                                     \
    const bf16_t* src = (8 * i <= m_last_ok) ? a_row0 + (int64_t)i * a_step : a_last; \
    g2l_16(src + (k0), &sA[buf][(wave * 64 + 8 * i) * BK]);                           \
  }
#define ISSUE_W(buf, k0)                                                              \
  _Pragma("unroll") for (int i = 0; i < 8; ++i)                                       \
    g2l_16(w_row0 + (int64_t)i * w_step + (k0), &sW[buf][(wave * 64 + 8 * i) * BK]);

  // ---- prologue: stage tile 0 ---------------------------------------------
  ISSUE_A(0, 0);
  if constexpr (WT == W_FP8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid >> 2) + 64 * i;
      rw[i] = *reinterpret_cast<const uint4*>(W8 + (int64_t)(n0 + row) * K + (tid & 3) * 16);
    }
  } else {
    ISSUE_W(0, 0);
  }
  if constexpr (WT == W_FP8) fp8_tile_to_lds(rw, &sW[0][0], tid);
  wait_vmem();
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int k1 = (kt + 1) * BK;
      ISSUE_A(buf ^ 1, k1);
      if constexpr (WT == W_FP8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = (tid >> 2) + 64 * i;
          rw[i] = *reinterpret_cast<const uint4*>(W8 + (int64_t)(n0 + row) * K + k1 + (tid & 3) * 16);
        }
      } else {
        ISSUE_W(buf ^ 1, k1);
      }
    }
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + fgrp;
      bf16x8_t wf[4], xf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rn = wn * 128 + i * 32 + frow;
        wf[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sW[buf][swz(rn, c)]));
        const int rm = wm * 128 + i * 32 + frow;
        xf[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(&sA[buf][swz(rm, c)]));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
    }
    if constexpr (WT == W_FP8) {
      if (more) fp8_tile_to_lds(rw, &sW[buf ^ 1][0], tid);
    }
    wait_vmem();
    __syncthreads();
  }
#undef ISSUE_A
#undef ISSUE_W

  // ---- epilogue ------------------------------------------------------------
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + wn * 128 + i * 32 + q * 8 + fgrp * 4;
      float4 bias = a.bias ? *reinterpret_cast<const float4*>(a.bias + n) : make_float4(0, 0, 0, 0);
      float4 scl = make_float4(1, 1, 1, 1);
      if constexpr (WT == W_FP8) scl = *reinterpret_cast<const float4*>(a.scale + n);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm * 128 + j * 32 + frow;
        if (m >= a.M) continue;
        float v0 = acc[i][j][q * 4 + 0] * scl.x + bias.x;
        float v1 = acc[i][j][q * 4 + 1] * scl.y + bias.y;
        float v2 = acc[i][j][q * 4 + 2] * scl.z + bias.z;
        float v3 = acc[i][j][q * 4 + 3] * scl.w + bias.w;
        if constexpr (EPI == EPI_GELU) {
          v0 = gelu_tanh_fast(round_bf16(v0));
          v1 = gelu_tanh_fast(round_bf16(v1));
          v2 = gelu_tanh_fast(round_bf16(v2));
          v3 = gelu_tanh_fast(round_bf16(v3));
        }
        if constexpr (EPI == EPI_RESID) {
          float4* r = reinterpret_cast<float4*>(a.R + (int64_t)m * a.ldr + n);
          float4 h = *r;
          h.x += round_bf16(v0);
          h.y += round_bf16(v1);
          h.z += round_bf16(v2);
          h.w += round_bf16(v3);
          *r = h;
        } else if constexpr (OUT_F32) {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.C) + (int64_t)m * a.ldc + n) =
              make_float4(v0, v1, v2, v3);
        } else {
          uint2 p;
          p.x = pack_bf16x2(v0, v1);
          p.y = pack_bf16x2(v2, v3);
          *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.C) + (int64_t)m * a.ldc + n) = p;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 GEMM (the fp32 check mode): 64 x 64 tile, BK = 16, 4 x 4 per thread.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs a) {
  __shared__ float sA[16][64 + 4];
  __shared__ float sW[16][64 + 4];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = tid & 15, ty = tid >> 4;
  const float* __restrict__ A = reinterpret_cast<const float*>(a.A);
  const float* __restrict__ Wt = reinterpret_cast<const float*>(a.W);
  float acc[4][4] = {};
  const int lr = tid >> 2, lk = (tid & 3) * 4;  // 64 rows x 16 k: 4 floats per thread
  for (int k0 = 0; k0 < a.K; k0 += 16) {
    {
      int m = m0 + lr;
      float4 v = make_float4(0, 0, 0, 0);
      if (m < a.M) {
        const float* p = A + (int64_t)m * a.lda + k0 + lk;
        if (k0 + lk + 3 < a.K) v = *reinterpret_cast<const float4*>(p);
        else {
          v.x = k0 + lk < a.K ? p[0] : 0.f;
          v.y = k0 + lk + 1 < a.K ? p[1] : 0.f;
          v.z = k0 + lk + 2 < a.K ? p[2] : 0.f;
        }
      }
      sA[lk][lr] = v.x; sA[lk + 1][lr] = v.y; sA[lk + 2][lr] = v.z; sA[lk + 3][lr] = v.w;
      int n = n0 + lr;
      float4 w = make_float4(0, 0, 0, 0);
      if (n < a.N) {
        const float* p = Wt + (int64_t)n * a.K + k0 + lk;
        if (k0 + lk + 3 < a.K) w = *reinterpret_cast<const float4*>(p);
        else {
          w.x = k0 + lk < a.K ? p[0] : 0.f;
          w.y = k0 + lk + 1 < a.K ? p[1] : 0.f;
          w.z = k0 + lk + 2 < a.K ? p[2] : 0.f;
        }
      }
      sW[lk][lr] = w.x; sW[lk + 1][lr] = w.y; sW[lk + 2][lr] = w.z; sW[lk + 3][lr] = w.w;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      float av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = sA[k][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = sW[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= a.N) continue;
      float v = acc[i][j] + (a.bias ? a.bias[n] : 0.f);
      if constexpr (EPI == EPI_GELU) v = gelu_tanh(v);
      if constexpr (EPI == EPI_RESID) {
        a.R[(int64_t)m * a.ldr + n] += v;
      } else {
        reinterpret_cast<float*>(a.C)[(int64_t)m * a.ldc + n] = v;
      }
    }
  }
}

template <int EPI, int WT, bool OUT_F32>
hipError_t launch_mfma(const GemmArgs& a, hipStream_t st) {
  const int num_tm = (a.M + BM - 1) / BM, num_tn = a.N / BN;
  hipLaunchKernelGGL((gemm_mfma_kernel<EPI, WT, OUT_F32>), dim3(num_tm * num_tn), dim3(NTHREADS),
                     0, st, a);
  return hipGetLastError();
}

}  // namespace

namespace allie {

bool gemm_mfma_supported(const GemmArgs& a) {
  return a.N % BN == 0 && a.K % BK == 0 && a.lda % 8 == 0 && a.M > 0;
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t st) {
  if (a.M == 0) return hipSuccess;
  if (a.wtype == W_F32) {
    dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
    switch (a.epi) {
      case EPI_STORE: hipLaunchKernelGGL(gemm_f32_kernel<EPI_STORE>, grid, dim3(256), 0, st, a); break;
      case EPI_GELU: hipLaunchKernelGGL(gemm_f32_kernel<EPI_GELU>, grid, dim3(256), 0, st, a); break;
      case EPI_RESID: hipLaunchKernelGGL(gemm_f32_kernel<EPI_RESID>, grid, dim3(256), 0, st, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (!gemm_mfma_supported(a)) return hipErrorInvalidValue;
  if (a.wtype == W_BF16) {
    switch (a.epi) {
      case EPI_STORE:
        return a.out_f32 ? launch_mfma<EPI_STORE, W_BF16, true>(a, st)
                         : launch_mfma<EPI_STORE, W_BF16, false>(a, st);
      case EPI_GELU: return launch_mfma<EPI_GELU, W_BF16, false>(a, st);
      case EPI_RESID: return launch_mfma<EPI_RESID, W_BF16, false>(a, st);
    }
  } else if (a.wtype == W_FP8) {
    switch (a.epi) {
      case EPI_STORE: return launch_mfma<EPI_STORE, W_FP8, false>(a, st);
      case EPI_GELU: return launch_mfma<EPI_GELU, W_FP8, false>(a, st);
      case EPI_RESID: return launch_mfma<EPI_RESID, W_FP8, false>(a, st);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace allie
