// Token embedding, LayerNorm and weight conversion kernels.
//
// Embedding follows CausalLMWithControlToken.forward (reference
// src/modeling/model.py:35-48) plus GPT-2's position add [lib]: Elo ids
// (id >= vocab) embed as [e, 1-e] @ control_embeds with
// e = (clamp(id - vocab, 500, 3000) - 500) / 2500, other ids as wte[id];
// then h = x + wpe[pos].  The residual stream h stays fp32 (under the
// reference's autocast the bf16 GEMM outputs are added to an fp32 stream).
// The first block's ln_1 is fused: the wave that owns a row has it in
// registers already.
//
// LayerNorm is GPT-2's (eps 1e-5, affine), statistics in fp32 with the
// two-pass variance over the register-resident row.  It can first add a bf16
// GEMM output to the fp32 residual row (h += y, the reference's residual add
// of a bf16 autocast projection) and write the sum back.  One wave per row; d is a
// multiple of 256 so each lane owns d/256 float4 groups.
#include "common.hpp"
#include "kernels.hpp"

namespace {

// Normalises the wave's register-resident row v and stores it as row `row`
// of y.  Gamma and beta are loaded group by group after the statistics, so
// the row costs few registers (an add + LayerNorm wave fits beside a
// persistent GEMM wave on one SIMD: that GEMM leaves 48-56 of 512 free).
template <int NV>
__device__ __forceinline__ void ln_row_store(const float4 (&v)[NV], int d, const float* __restrict__ g,
                                             const float* __restrict__ b, float eps, void* y, int64_t row,
                                             int act_bf16) {
  const int lane = threadIdx.x & 63;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mean = wave_sum(s) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, e = v[i].w - mean;
    q += (a * a + b * b) + (c * c + e * e);
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)d + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 4;
    const float4 gg = *reinterpret_cast<const float4*>(g + c);
    const float4 bb = *reinterpret_cast<const float4*>(b + c);
    float o0 = (v[i].x - mean) * rstd * gg.x + bb.x;
    float o1 = (v[i].y - mean) * rstd * gg.y + bb.y;
    float o2 = (v[i].z - mean) * rstd * gg.z + bb.z;
    float o3 = (v[i].w - mean) * rstd * gg.w + bb.w;
    if (act_bf16) {
      uint2 p;
      p.x = pack_bf16x2(o0, o1);
      p.y = pack_bf16x2(o2, o3);
      *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(y) + row * d + c) = p;
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + row * d + c) = make_float4(o0, o1, o2, o3);
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void embed_ln_kernel(allie::EmbedArgs a) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const int lane = threadIdx.x & 63;
  const int d = a.d;
  const int id = a.ids[t];
  int p = a.pos[t];  // out-of-range positions are flagged by the caller; never read past wpe
  p = p < 0 ? 0 : (p >= a.n_positions ? a.n_positions - 1 : p);
  const bool elo = id >= a.vocab;
  float e = 0.f, e1 = 0.f;
  if (elo) {
    int r = id - a.vocab;
    r = r < 500 ? 500 : (r > 3000 ? 3000 : r);
    e = (float)(r - 500) / 2500.0f;
    e1 = 1.0f - e;
    if (a.act_bf16) {  // autocast: the [e, 1-e] @ Wc matmul runs in bf16
      e = round_bf16(e);
      e1 = round_bf16(e1);
    }
  }
  const int row = id < 0 ? 0 : (id > a.vocab - 1 ? a.vocab - 1 : id);
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 4;
    float4 x;
    if (elo) {
      float4 c0 = *reinterpret_cast<const float4*>(a.ctrl + c);
      float4 c1 = *reinterpret_cast<const float4*>(a.ctrl + d + c);
      if (a.act_bf16) {
        x.x = round_bf16(e * round_bf16(c0.x) + e1 * round_bf16(c1.x));
        x.y = round_bf16(e * round_bf16(c0.y) + e1 * round_bf16(c1.y));
        x.z = round_bf16(e * round_bf16(c0.z) + e1 * round_bf16(c1.z));
        x.w = round_bf16(e * round_bf16(c0.w) + e1 * round_bf16(c1.w));
      } else {
        x.x = e * c0.x + e1 * c1.x;
        x.y = e * c0.y + e1 * c1.y;
        x.z = e * c0.z + e1 * c1.z;
        x.w = e * c0.w + e1 * c1.w;
      }
    } else {
      x = *reinterpret_cast<const float4*>(a.wte + (int64_t)row * d + c);
    }
    float4 pe = *reinterpret_cast<const float4*>(a.wpe + (int64_t)p * d + c);
    v[i] = make_float4(x.x + pe.x, x.y + pe.y, x.z + pe.z, x.w + pe.w);
    *reinterpret_cast<float4*>(a.h + t * d + c) = v[i];
  }
  ln_row_store<NV>(v, d, a.ln_g, a.ln_b, a.eps, a.x, t, a.act_bf16);
}

// ADD: 0 no addend, 1 add, 2 add and add2 (template arguments, so that the
// row's loads are issued together: loads under a runtime condition each get
// a wait of their own)
template <int NV, int ADD>
__global__ __launch_bounds__(256) void layernorm_kernel(allie::LNArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  if (r >= a.rows_out) return;
  const int lane = threadIdx.x & 63;
  const int d = a.d;
  if (r >= a.rows) {  // padding rows of a gathered batch
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 4;
      if (a.act_bf16)
        *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.y) + r * d + c) = make_uint2(0, 0);
      else
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.y) + r * d + c) =
            make_float4(0, 0, 0, 0);
    }
    return;
  }
  const int64_t src = a.row_idx ? (int64_t)a.row_idx[r] : r;
  float4 v[NV];
  uint2 y[NV], z[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 64 + lane) * 4;
    v[i] = *reinterpret_cast<const float4*>(a.h + src * d + c);
    if constexpr (ADD >= 1) y[i] = *reinterpret_cast<const uint2*>(reinterpret_cast<const bf16_t*>(a.add) + src * d + c);
    if constexpr (ADD >= 2) z[i] = *reinterpret_cast<const uint2*>(reinterpret_cast<const bf16_t*>(a.add2) + src * d + c);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if constexpr (ADD >= 1) {  // h + bf16 GEMM output, in fp32 (exact widening)
      v[i].x += bf2f(y[i].x & 0xffffu);
      v[i].y += bf2f(y[i].x >> 16);
      v[i].z += bf2f(y[i].y & 0xffffu);
      v[i].w += bf2f(y[i].y >> 16);
    }
    if constexpr (ADD >= 2) {
      v[i].x += bf2f(z[i].x & 0xffffu);
      v[i].y += bf2f(z[i].x >> 16);
      v[i].z += bf2f(z[i].y & 0xffffu);
      v[i].w += bf2f(z[i].y >> 16);
    }
  }
  if (a.h_out) {
#pragma unroll
    for (int i = 0; i < NV; ++i) *reinterpret_cast<float4*>(a.h_out + src * d + (i * 64 + lane) * 4) = v[i];
  }
  ln_row_store<NV>(v, d, a.g, a.b, a.eps, a.y, r, a.act_bf16);
}

// dst row r = src row idx[r], 16 bytes per thread
__global__ __launch_bounds__(256) void gather_rows_kernel(const char* __restrict__ src, const int32_t* __restrict__ idx,
                                                          int row_bytes, char* __restrict__ dst) {
  const int64_t r = blockIdx.x;
  const int64_t s = idx[r];
  for (int c = threadIdx.x * 16; c < row_bytes; c += 256 * 16)
    *reinterpret_cast<uint4*>(dst + r * row_bytes + c) = *reinterpret_cast<const uint4*>(src + s * row_bytes + c);
}

__global__ void transpose_convert_kernel(const float* __restrict__ src, int rows, int cols,
                                         void* dst, int dst_bf16, int ld_dst) {
  // src [rows][cols] -> dst[c][r] (ld_dst = row stride of dst)
  __shared__ float tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 32 x 8
  for (int j = ty; j < 32; j += 8) {
    int r = r0 + j, c = c0 + tx;
    tile[j][tx] = (r < rows && c < cols) ? src[(int64_t)r * cols + c] : 0.f;
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    int c = c0 + j, r = r0 + tx;
    if (c < cols && r < rows) {
      float v = tile[tx][j];
      if (dst_bf16)
        reinterpret_cast<bf16_t*>(dst)[(int64_t)c * ld_dst + r] = (bf16_t)f2bf(v);
      else
        reinterpret_cast<float*>(dst)[(int64_t)c * ld_dst + r] = v;
    }
  }
}

__global__ void convert_kernel(const float* __restrict__ src, int64_t n, void* dst, int dst_bf16,
                               int round_only) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = src[i];
    if (dst_bf16)
      reinterpret_cast<bf16_t*>(dst)[i] = (bf16_t)f2bf(v);
    else
      reinterpret_cast<float*>(dst)[i] = round_only ? round_bf16(v) : v;
  }
}

}  // namespace

namespace allie {

#define ALLIE_NV_SWITCH(NVAL, ...)   \
  switch (NVAL) {                    \
    case 1: { constexpr int NV = 1; __VA_ARGS__; } break; \
    case 2: { constexpr int NV = 2; __VA_ARGS__; } break; \
    case 3: { constexpr int NV = 3; __VA_ARGS__; } break; \
    case 4: { constexpr int NV = 4; __VA_ARGS__; } break; \
    case 5: { constexpr int NV = 5; __VA_ARGS__; } break; \
    case 6: { constexpr int NV = 6; __VA_ARGS__; } break; \
    case 8: { constexpr int NV = 8; __VA_ARGS__; } break; \
    default: return hipErrorInvalidValue; \
  }

hipError_t launch_embed_ln(const EmbedArgs& a, hipStream_t st) {
  if (a.d % 256 != 0) return hipErrorInvalidValue;
  if (a.T == 0) return hipSuccess;
  dim3 grid((a.T + 3) / 4);
  ALLIE_NV_SWITCH(a.d / 256, hipLaunchKernelGGL(embed_ln_kernel<NV>, grid, dim3(256), 0, st, a));
  return hipGetLastError();
}

hipError_t launch_layernorm(const LNArgs& a, hipStream_t st) {
  if (a.d % 256 != 0 || a.rows_out < a.rows) return hipErrorInvalidValue;
  if ((a.add && !a.act_bf16) || (a.add2 && !a.add)) return hipErrorInvalidValue;
  if (a.rows_out == 0) return hipSuccess;
  dim3 grid((a.rows_out + 3) / 4);
  switch (a.add ? (a.add2 ? 2 : 1) : 0) {
    case 0: ALLIE_NV_SWITCH(a.d / 256, hipLaunchKernelGGL((layernorm_kernel<NV, 0>), grid, dim3(256), 0, st, a)); break;
    case 1: ALLIE_NV_SWITCH(a.d / 256, hipLaunchKernelGGL((layernorm_kernel<NV, 1>), grid, dim3(256), 0, st, a)); break;
    default: ALLIE_NV_SWITCH(a.d / 256, hipLaunchKernelGGL((layernorm_kernel<NV, 2>), grid, dim3(256), 0, st, a)); break;
  }
  return hipGetLastError();
}

hipError_t launch_gather_rows(const void* src, const int32_t* idx, int rows, int row_bytes, void* dst,
                              hipStream_t st) {
  if (row_bytes % 16 != 0 || rows < 0) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)rows), dim3(256), 0, st, static_cast<const char*>(src), idx,
                     row_bytes, static_cast<char*>(dst));
  return hipGetLastError();
}

hipError_t launch_transpose_convert(const float* src, int rows, int cols, void* dst, int dst_bf16,
                                    int ld_dst, hipStream_t st) {
  dim3 grid((cols + 31) / 32, (rows + 31) / 32);
  hipLaunchKernelGGL(transpose_convert_kernel, grid, dim3(256), 0, st, src, rows, cols, dst,
                     dst_bf16, ld_dst);
  return hipGetLastError();
}

hipError_t launch_convert(const float* src, int64_t n, void* dst, int dst_bf16, int round_bf16,
                          hipStream_t st) {
  if (n == 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(convert_kernel, dim3((unsigned)blocks), dim3(256), 0, st, src, n, dst,
                     dst_bf16, round_bf16);
  return hipGetLastError();
}

}  // namespace allie
