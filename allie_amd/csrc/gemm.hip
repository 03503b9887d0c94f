// GEMMs of the transformer blocks and the heads on gfx950.
//
// C[m, n] = sum_k A[m, k] * W[n, k] with both operands K-contiguous: A is the
// activation stream [T][K] (bf16), W the weight matrix [N][K] (bf16, or fp8
// e4m3 with a per-output-channel fp32 scale).  This is the Conv1D
// ``addmm(b, x, W[in,out])`` of GPT-2 [lib transformers Conv1D] with the
// weights repacked once to [out][in] at load time.
//
// MFMA kernel: 256 threads (4 waves, 2 (m) x 2 (n)), block tile 256 (m) x 128
// (n) -- or 192 / 128 rows when M is small (gemm_tile_m) -- two blocks per
// CU.  Each wave owns a 128 (m) x 64 (n) sub-tile = 2 x 4
// MFMA 32x32x16 bf16 blocks (128 fp32 accumulators), which leaves room for a
// second block on every SIMD: while one block sits in its epilogue, prologue
// or a barrier, the other keeps the matrix cores busy.  (Measured on the
// 53205 x 4096 x 1024 MLP GEMM with one 256 x 256 block per CU: prologue 7K,
// k-loop 58K and epilogue 25-75K cycles per tile, the epilogues of all CUs
// falling together and idling the MFMAs.)
//
// k-tiles of BK = 32 go through a ring of STAGES LDS buffers filled by direct
// global->LDS 16-byte loads; the ring is waited with partial vmcnt counts and
// a fence-free s_barrier (a __syncthreads() fence would drain every
// outstanding load).
//
// The MFMA's first operand is the weight fragment and its second the
// activation fragment, so each lane's accumulator holds 4 consecutive output
// columns of one row.
//
// k order inside a k-tile: in MFMA step s (0, 1) the lanes of half h = lane/32
// multiply k = 16 h + 8 s .. +7.  Both operands use this order, so the sum is
// unchanged, and it lets an fp8 weight row hand a lane both of its steps' k
// values as one 16-byte chunk.
//
// LDS layouts (gfx950 LDS: 64 banks x 4 B, a 16-byte read serves 16 lanes per
// clock, so 16 consecutive rows must hit 16 distinct 16-byte slots of a
// 256-byte window):
//   bf16 rows of 64 B (4 chunks):  chunk c of row r at c ^ ((r >> 2) & 3)
//   fp8  rows of 32 B (2 chunks):  chunk c of row r at c ^ ((r >> 3) & 1)
// Fragment reads are double-buffered in registers: the reads of step s + 1 are
// issued while the MFMAs of step s run.
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
// with fp32 output (no rounding) when out_f32 is set (heads).  fp8 weights:
// acc is multiplied by the output channel's scale before the bias.  bf16
// results are transposed through LDS so global memory sees 128-byte rows.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace {

using namespace allie;

constexpr int BM = 256, BN = 128, BK = 32;
constexpr int STAGES = 3;
constexpr int NTHREADS = 256;
constexpr int FM = 4, FN = 2;     // 32x32 MFMA blocks per wave along m and n
constexpr int GROUP_M = 4;
constexpr int A_STAGE = BM * BK;  // bf16 elements per A stage (16 KiB)
constexpr int W_STAGE = BN * BK;  // bf16 elements per W stage (8 KiB; fp8 uses half)
constexpr int EP = 72;            // epilogue transpose row pitch (bf16): 64 + 8 pad
static_assert(4 * 128 * EP <= STAGES * (A_STAGE + W_STAGE), "epilogue region fits the ring");

// element offset of logical 16-byte chunk c of row r in a bf16 stage
ALLIE_DEV int swz16(int r, int c) { return r * BK + ((c ^ ((r >> 2) & 3)) << 3); }
// byte offset of logical 16-byte chunk c of row r in an fp8 stage
ALLIE_DEV int swz8(int r, int c) { return r * BK + ((c ^ ((r >> 3) & 1)) << 4); }

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

typedef __attribute__((address_space(3))) void lds_void_t;

// Direct global -> LDS copy of 16 bytes per lane: the wave writes 1 KiB of
// LDS contiguously at `lds` (lane i at lds + 16 i).
ALLIE_DEV void g2l_16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 16, 0, 0);
}

// Wait until at most n_tiles k-tiles' worth (VMT instructions each) of this
// wave's vector-memory operations are pending; the oldest complete first.
template <int VMT>
ALLIE_DEV void wait_vm_tiles(int n_tiles) {
  switch (n_tiles) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(VMT) : "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * VMT) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * VMT) : "memory"); break;
  }
}
static_assert(STAGES - 1 <= 3, "wait_vm_tiles covers up to three newer tiles in flight");

// Workgroup barrier without a memory fence: LDS reads issued before it have
// completed (lgkmcnt(0)); the compiler may not move memory accesses across it.
ALLIE_DEV void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Scheduling hint for one k-step (the next step's NR fragment reads and this
// step's NM MFMAs): one LDS read after each early MFMA, so the reads are
// issued early and the remaining MFMAs cover their latency.
template <int NR, int NM>
ALLIE_DEV void interleave_step() {
  static_assert(NR <= NM, "one read per MFMA at most");
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
  }
  if (NM > NR) __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
}

// 8 fp8 e4m3 (two dwords) -> 8 bf16 packed in 4 dwords (exact).
ALLIE_DEV u32x4_t fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  u32x4_t o;
  o.x = fp8e4m3_to_bf16(lo & 0xffu) | (fp8e4m3_to_bf16((lo >> 8) & 0xffu) << 16);
  o.y = fp8e4m3_to_bf16((lo >> 16) & 0xffu) | (fp8e4m3_to_bf16(lo >> 24) << 16);
  o.z = fp8e4m3_to_bf16(hi & 0xffu) | (fp8e4m3_to_bf16((hi >> 8) & 0xffu) << 16);
  o.w = fp8e4m3_to_bf16((hi >> 16) & 0xffu) | (fp8e4m3_to_bf16(hi >> 24) << 16);
  return o;
}

// output of the MFMA kernel: bf16 through LDS, fp32 rows (heads), or the
// fp32 partial sums of one K split (reduced by splitk_reduce_kernel)
enum { OUT_BF16 = 0, OUT_F32 = 1, OUT_PART = 2 };
// fp8 weights already widened to bf16 (exact) in the call's wdq buffer:
// loaded as bf16, scaled per output channel as fp8 weights are
constexpr int W_FP8W = 3;

template <int EPI, int WT, int OUT, int BMT>
__global__ __launch_bounds__(NTHREADS, 2) void gemm_mfma_kernel(GemmArgs a) {
  // block tile BMT (128, 192 or 256) x BN; wave (wm, wn) owns WMX x 64
  constexpr int FMT = BMT / 64, WMX = BMT / 2, ASTG = BMT * BK, AI = BMT / 64;
  constexpr int STG = BMT == 128 ? 4 : STAGES;  // ring stages (128-row tiles: one more in flight)
  static_assert(4 * WMX * EP <= STG * (ASTG + W_STAGE), "epilogue region fits the ring");
  // one LDS arena: the ring of A stages, the ring of W stages; the epilogue
  // reuses it to transpose the output tile
  __shared__ __attribute__((aligned(1024))) bf16_t smem[STG * (ASTG + W_STAGE)];
  auto sA = [&](int s) { return smem + s * ASTG; };
  auto sW = [&](int s) { return smem + STG * ASTG + s * W_STAGE; };
  // fp8 weights come as bytes (FP8) or widened to bf16 (W_FP8W, loaded as
  // bf16); either way the sum is scaled per output channel (SCALED)
  constexpr bool FP8 = WT == W_FP8;
  constexpr bool SCALED = WT == W_FP8 || WT == W_FP8W;
  // vector-memory instructions per wave per k-tile: A BMT / 64, W 2 (bf16) or 1 (fp8)
  constexpr int VMT = AI + (FP8 ? 1 : 2);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (LDS-DMA base)
  constexpr bool PART = OUT == OUT_PART;
  const int num_tm = (a.M + BMT - 1) / BMT, num_tn = a.N / BN;
  // K splits: block b computes split b / tiles of tile b % tiles
  const int n_tiles = PART ? gridDim.x / a.split : gridDim.x;
  const int split_id = PART ? blockIdx.x / n_tiles : 0;
  int tm, tn;
  tile_coords(PART ? blockIdx.x - split_id * n_tiles : blockIdx.x, n_tiles, num_tm, num_tn, tm, tn);
  const int m0 = tm * BMT, n0 = tn * BN;
  const int K = a.K;
  const int KT = K / BK / (PART ? a.split : 1);  // k-tiles of this block
  const int k_begin = split_id * KT * BK;

  // ---- loader geometry ----------------------------------------------------
  // bf16 rows of 64 B, 16 rows per DMA instruction: lane -> row lane / 4,
  // physical chunk lane % 4, which holds logical chunk (lane % 4) ^ ((row >> 2) & 3).
  // A: wave w fills rows [BMT/4 w, BMT/4 (w + 1)) (AI instructions); W: rows
  // [32 w, 32 w + 32) (2 instructions).
  const int lr16 = lane >> 2;
  const int lc16 = (lane & 3) ^ ((lr16 >> 2) & 3);
  const bf16_t* __restrict__ A = reinterpret_cast<const bf16_t*>(a.A);
  // rows at or past M read the last valid row instead (results discarded)
  const bf16_t* a_src[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    int m = m0 + wave * (BMT / 4) + 16 * i + lr16;
    m = m < a.M ? m : a.M - 1;
    a_src[i] = A + (int64_t)m * a.lda + lc16 * 8 + k_begin;
  }
  const bf16_t* __restrict__ Wb = reinterpret_cast<const bf16_t*>(a.W);
  const bf16_t* w_src = Wb + (int64_t)(n0 + wave * 32 + lr16) * K + lc16 * 8 + k_begin;
  const int64_t w_step16 = (int64_t)16 * K;
  // fp8 rows of 32 B, 32 rows per DMA instruction: lane -> row lane / 2,
  // physical chunk lane % 2; wave w fills rows [32 w, 32 w + 32).
  const int lr8 = lane >> 1;
  const int lc8 = (lane & 1) ^ ((lr8 >> 3) & 1);
  const uint8_t* __restrict__ W8 = reinterpret_cast<const uint8_t*>(a.W);
  const uint8_t* w8_src = W8 + (int64_t)(n0 + wave * 32 + lr8) * K + lc8 * 16 + k_begin;

  auto issue = [&](int kt, int s) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < AI; ++i) g2l_16(a_src[i] + k0, sA(s) + (wave * (BMT / 4) + 16 * i) * BK);
    if constexpr (FP8) {
      g2l_16(w8_src + k0, reinterpret_cast<uint8_t*>(sW(s)) + wave * 32 * BK);
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) g2l_16(w_src + i * w_step16 + k0, sW(s) + (wave * 32 + 16 * i) * BK);
    }
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int frow = lane & 31, half = lane >> 5;
  const int n_base = n0 + wn * 64;

  // accumulator element (i, j, q, e) is output (m, n) with
  // m = m0 + wm WMX + j 32 + frow, n = n_base + i 32 + q 8 + half 4 + e.
  // bf16 weights: the accumulators start at the bias (fp8 weights scale the
  // sum first, so their bias is added in the epilogue; K splits add it in
  // the reduction).
  f32x16_t acc[FN][FMT];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    f32x16_t init{};
    if (!SCALED && !PART && a.bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 b = *reinterpret_cast<const float4*>(a.bias + n_base + i * 32 + q * 8 + half * 4);
        init[q * 4 + 0] = b.x;
        init[q * 4 + 1] = b.y;
        init[q * 4 + 2] = b.z;
        init[q * 4 + 3] = b.w;
      }
    }
#pragma unroll
    for (int j = 0; j < FMT; ++j) acc[i][j] = init;
  }

  // fragments of step `st` of the k-tile in stage s
  auto load_a = [&](int s, int st, bf16x8_t(&xf)[FMT]) {
    const int c = 2 * half + st;
#pragma unroll
    for (int j = 0; j < FMT; ++j) {
      const int r = wm * WMX + j * 32 + frow;
      xf[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(sA(s) + swz16(r, c)));
    }
  };
  auto load_w = [&](int s, int st, bf16x8_t(&wf)[FN]) {
    const int c = 2 * half + st;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int r = wn * 64 + i * 32 + frow;
      wf[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(sW(s) + swz16(r, c)));
    }
  };
  // fp8: one 16-byte read per weight fragment row holds both steps
  auto load_w8 = [&](int s, u32x4_t(&wq)[FN]) {
    const uint8_t* base = reinterpret_cast<const uint8_t*>(sW(s));
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int r = wn * 64 + i * 32 + frow;
      wq[i] = *reinterpret_cast<const u32x4_t*>(base + swz8(r, half));
    }
  };
  auto widen_w8 = [&](const u32x4_t(&wq)[FN], int st, bf16x8_t(&wf)[FN]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
      wf[i] = __builtin_bit_cast(bf16x8_t, st == 0 ? fp8x8_to_bf16x8(wq[i].x, wq[i].y)
                                                   : fp8x8_to_bf16x8(wq[i].z, wq[i].w));
  };
  auto mfma_step = [&](const bf16x8_t(&wf)[FN], const bf16x8_t(&xf)[FMT]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FMT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
  };
  constexpr int NMF = FN * FMT;  // MFMAs per step

  // ---- prologue: fill the ring (tile 0 must land) ---------------------------
  const int n_pre = KT < STG ? KT : STG;
  for (int t = 0; t < n_pre; ++t) issue(t, t);
  wait_vm_tiles<VMT>(n_pre - 1);
  lds_barrier();

  bf16x8_t wP[FN], xP[FMT], wQ[FN], xQ[FMT];
  u32x4_t w8[FN];
  if constexpr (FP8) {
    load_w8(0, w8);
    load_a(0, 0, xP);
    widen_w8(w8, 0, wP);
  } else {
    load_w(0, 0, wP);
    load_a(0, 0, xP);
  }

  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt % STG;
    const int s1 = (kt + 1) % STG;
    // step 0: read step 1's fragments, multiply step 0's
    if constexpr (FP8) {
      widen_w8(w8, 1, wQ);
      load_a(s, 1, xQ);
      mfma_step(wP, xP);
      interleave_step<FMT, NMF>();
    } else {
      load_w(s, 1, wQ);
      load_a(s, 1, xQ);
      mfma_step(wP, xP);
      interleave_step<FN + FMT, NMF>();
    }
    // step 1: tile kt + 1 must have landed; then recycle stage s for tile
    // kt + STG and read the next tile's first fragments
    {
      int newer = KT - kt - 2;
      newer = newer < STG - 2 ? newer : STG - 2;
      wait_vm_tiles<VMT>(newer > 0 ? newer : 0);
    }
    lds_barrier();
    if (kt + STG < KT) issue(kt + STG, s);
    // after the last tile these read a stale (in-bounds) stage, never used
    if constexpr (FP8) {
      load_w8(s1, w8);
      load_a(s1, 0, xP);
      mfma_step(wQ, xQ);
      interleave_step<FN + FMT, NMF>();
      widen_w8(w8, 0, wP);
    } else {
      load_w(s1, 0, wP);
      load_a(s1, 0, xP);
      mfma_step(wQ, xQ);
      interleave_step<FN + FMT, NMF>();
    }
  }

  // ---- epilogue ------------------------------------------------------------
  if constexpr (OUT != OUT_BF16) {
    // heads (small M) and K-split partials: direct 16-byte stores of fp32
    // rows (the heads' bias already in acc)
    float* Cf = PART ? a.part + (int64_t)split_id * a.M * a.N : reinterpret_cast<float*>(a.C);
    const int64_t ldc = PART ? a.N : a.ldc;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n_base + i * 32 + q * 8 + half * 4;
#pragma unroll
        for (int j = 0; j < FMT; ++j) {
          const int m = m0 + wm * WMX + j * 32 + frow;
          if (m >= a.M) continue;
          *reinterpret_cast<float4*>(Cf + (int64_t)m * ldc + n) =
              make_float4(acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
        }
      }
    }
  } else {
    // bf16 results go through LDS so that global memory sees whole 128-byte
    // row segments: each wave writes its WMX (m) x 64 (n) sub-tile into a
    // private region of rows padded to EP bf16, then reads it back 16 bytes
    // per lane, 8 lanes per row.
    lds_barrier();  // every wave is done with the ring
    bf16_t* reg = smem + wave * WMX * EP;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = i * 32 + q * 8 + half * 4;  // column inside the sub-tile
        float4 bias = make_float4(0, 0, 0, 0), scl = make_float4(1, 1, 1, 1);
        if constexpr (SCALED) {
          if (a.bias) bias = *reinterpret_cast<const float4*>(a.bias + n_base + nl);
          scl = *reinterpret_cast<const float4*>(a.scale + n_base + nl);
        }
#pragma unroll
        for (int j = 0; j < FMT; ++j) {
          const int ml = j * 32 + frow;
          float v0 = acc[i][j][q * 4 + 0], v1 = acc[i][j][q * 4 + 1];
          float v2 = acc[i][j][q * 4 + 2], v3 = acc[i][j][q * 4 + 3];
          if constexpr (SCALED) {
            v0 = v0 * scl.x + bias.x;
            v1 = v1 * scl.y + bias.y;
            v2 = v2 * scl.z + bias.z;
            v3 = v3 * scl.w + bias.w;
          }
          if constexpr (EPI == EPI_GELU) {
            // gelu_new of the bf16 addmm result
            round_bf16x2(v0, v1);
            round_bf16x2(v2, v3);
            v0 = gelu_tanh_fast(v0);
            v1 = gelu_tanh_fast(v1);
            v2 = gelu_tanh_fast(v2);
            v3 = gelu_tanh_fast(v3);
          }
          uint2 p;
          p.x = pack_bf16x2(v0, v1);
          p.y = pack_bf16x2(v2, v3);
          *reinterpret_cast<uint2*>(reg + ml * EP + nl) = p;
        }
      }
    }
    // read back: lane -> row (lane / 8) + 8 it, columns 8 (lane % 8) .. +7
    const int cl = (lane & 7) * 8;
    if constexpr (EPI == EPI_RESID) {
      // R += the bf16-rounded value (exact in fp32).  All loads of R for 8
      // rows are issued before any store: a store may alias the next load, so
      // interleaving them would expose the memory latency 16 times.
      float* __restrict__ Rp = a.R;
      constexpr int RG = WMX / 8;  // groups of 8 rows, 8 at a time
#pragma unroll
      for (int half8 = 0; half8 < (RG + 7) / 8; ++half8) {
        uint4 v[8];
        float4 h0[8], h1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (half8 * 8 + u >= RG) break;
          const int ml = (half8 * 8 + u) * 8 + (lane >> 3);
          const int m = m0 + wm * WMX + ml;
          v[u] = *reinterpret_cast<const uint4*>(reg + ml * EP + cl);
          if (m < a.M) {
            const float4* r = reinterpret_cast<const float4*>(Rp + (int64_t)m * a.ldr + n_base + cl);
            h0[u] = r[0];
            h1[u] = r[1];
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (half8 * 8 + u >= RG) break;
          const int ml = (half8 * 8 + u) * 8 + (lane >> 3);
          const int m = m0 + wm * WMX + ml;
          if (m >= a.M) continue;
          float4 x0 = h0[u], x1 = h1[u];
          x0.x += bf2f(v[u].x & 0xffffu); x0.y += bf2f(v[u].x >> 16);
          x0.z += bf2f(v[u].y & 0xffffu); x0.w += bf2f(v[u].y >> 16);
          x1.x += bf2f(v[u].z & 0xffffu); x1.y += bf2f(v[u].z >> 16);
          x1.z += bf2f(v[u].w & 0xffffu); x1.w += bf2f(v[u].w >> 16);
          float4* r = reinterpret_cast<float4*>(Rp + (int64_t)m * a.ldr + n_base + cl);
          r[0] = x0;
          r[1] = x1;
        }
      }
    } else if (EPI == EPI_STORE && a.kv_pool && n_base >= a.N / 3) {
      // an extend's keys and values: this wave's 64 columns are one head's
      // key or value; row m goes to its pool slot (16 positions per block)
      const int d = a.N / 3, H = d / 64;
      const int kvi = n_base >= 2 * d ? 1 : 0, head = (n_base - (kvi + 1) * d) / 64;
      bf16_t* pl = reinterpret_cast<bf16_t*>(a.kv_pool) + ((int64_t)a.kv_layer * a.kv_pool_blocks * 2 + kvi) * H * 1024 +
                   (int64_t)head * 1024 + cl;
#pragma unroll 4
      for (int it = 0; it < WMX / 8; ++it) {
        const int ml = it * 8 + (lane >> 3);
        const int m = m0 + wm * WMX + ml;
        const uint4 v = *reinterpret_cast<const uint4*>(reg + ml * EP + cl);
        if (m >= a.M) continue;
        const int sl = a.kv_slot[m];
        if (sl < 0 || (sl >> 4) >= a.kv_pool_blocks) continue;
        *reinterpret_cast<uint4*>(pl + ((int64_t)(sl >> 4) * 2 * H * 16 + (sl & 15)) * 64) = v;
      }
    } else {
#pragma unroll 4
      for (int it = 0; it < WMX / 8; ++it) {
        const int ml = it * 8 + (lane >> 3);
        const int m = m0 + wm * WMX + ml;
        const uint4 v = *reinterpret_cast<const uint4*>(reg + ml * EP + cl);
        if (m >= a.M) continue;
        *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(a.C) + (int64_t)m * a.ldc + n_base + cl) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large GEMMs (the prefill's QKV, attention c_proj, c_fc and MLP c_proj over
// tens of thousands of tokens, bf16 weights, bf16 output): a persistent
// kernel, one block of 4 waves per CU, block tile 256 (m) x 256 (n).  Each
// wave owns 128 x 128 = 4 x 4 MFMA 32x32x16 blocks; its 256 fp32
// accumulators live in the accumulation registers (one wave per SIMD has 512
// registers).  Against the 256 x 128 kernel above, a tile moves 128 instead
// of 85 FLOP per byte through L2, and a wave issues 8 fragment reads per 16
// MFMAs instead of 6 per 8.
//
// k-tiles of 64: every row of a stage is one whole 128-byte line of A or W,
// so each request fetches a full line.  Two stages (128 KiB): tile kt + 2
// loads while tiles kt and kt + 1 are multiplied, its W rows during k-step 1
// (a wave reads all four k-steps' W fragments in k-step 0, so after a
// barrier the stage's W rows are free) and its A rows during k-step 3.
// Issuing a whole k-tile's 16 loads per wave at one point stalled MFMA issue
// for ~1300 cycles per k-tile while the texture unit drained them (measured
// with s_memtime stamps: 3500 cycles per k-tile against 2400 without
// loads); split in two they hide behind the MFMAs.  The loads are buffer
// loads straight to LDS over the tile's own rows: rows past M read as 0, the
// row is in the per-lane offset and the k offset in the scalar one.
//
// Persistent tile loop: a tile's last two k-tiles refill their stages with
// the next tile's first two k-tiles (and its bias and scale slices), so
// these load under the last MFMAs and the epilogue (C2 forward 37.3 -> 36.8
// ms; with an odd k-tile count they are requested after the last k-tile).
// The epilogue goes through a separate wave-private
// LDS region in chunks of 32 rows x 64 columns (rows of 128 bytes to global
// memory) with buffer stores, which are always issued (rows past M fall
// outside the buffer and are dropped), so every wave has exactly STORES
// stores in flight when the next tile's waits count its loads.
//
// k order inside a k-tile: in MFMA step s (0..3) the lanes of half h multiply
// logical chunk 2 s + h (k = 16 s + 8 h .. +7), identically for both
// operands.  LDS rows of 128 B (8 chunks): chunk c of row r sits at
// c ^ ((r >> 1) & 7), so 16 consecutive rows reading one chunk hit 16
// distinct 16-byte bank groups (rows r and r + 1 fill opposite halves of the
// 64 banks).  Epilogues: EPI_STORE C = bf16(acc + b), EPI_GELU
// C = bf16(gelu(bf16(acc + b))).
namespace big {
constexpr int BM = 256, BN = 256, BK = 64, STAGES = 2;
constexpr int FM = 4, FN = 4;       // 32x32 MFMA blocks per wave along m and n
constexpr int A_STAGE = BM * BK;    // bf16 elements per stage (32 KiB each)
constexpr int W_STAGE = BN * BK;
constexpr int RING = STAGES * (A_STAGE + W_STAGE);  // 128 KiB
constexpr int DMA = 8;              // DMA instructions per wave per k-tile and operand
constexpr int EP = 72;              // epilogue chunk row pitch (bf16)
constexpr int CHUNK = 32 * EP;      // one wave's epilogue region (bf16 elements)
// a tile's 256 fp32 bias values and 256 fp32 weight scales, in two slots by
// tile parity (the next tile's land while this one's epilogue reads its
// own), then a spare slot that absent ones are loaded into (bf16 elements)
constexpr int BIAS = RING + 4 * CHUNK;
constexpr int SCALE = BIAS + 2 * BN;
constexpr int SLOT = 4 * BN;            // parity stride
constexpr int SPARE = BIAS + 2 * SLOT;
constexpr int SMEM = SPARE + 2 * BN;    // 152 KiB
constexpr int STORES = 32;          // epilogue stores per wave per tile

// element offset of logical 16-byte chunk c of row r in a stage
ALLIE_DEV int swz(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 7)) << 3); }

// s_waitcnt vmcnt(N): at most N of this wave's vector-memory operations in flight
template <int N>
ALLIE_DEV void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
}  // namespace big

typedef __attribute__((address_space(3))) void lds_void_t2;

// Scheduling hint for a k-step of the persistent kernel: its NM MFMAs with,
// after the first ones, NR fragment reads, NW LDS writes and (every
// NM / NV MFMAs) NV loads.
template <int NR, int NW, int NV, int NM>
ALLIE_DEV void interleave_rwl() {
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
    if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    if (i < NW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    if (NV > 0 && i % (NM / (NV > 0 ? NV : 1)) == 0 && i / (NM / (NV > 0 ? NV : 1)) < NV)
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);            // VMEM read
  }
}

// The value unchanged, but opaque to the optimizer: keeps address arithmetic
// inside the tile loop instead of dozens of hoisted registers.
ALLIE_DEV int opaque_s(int v) {
  asm volatile("" : "+s"(v));
  return v;
}
ALLIE_DEV int opaque_v(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
// LDS reads the compiler's wait insertion does not track, each statement
// with its own wait (lgkmcnt(0)) so that no use or copy of a result can be
// placed between a read and the wait.  Used where the compiler would
// otherwise wait for every outstanding LDS DMA load.
// 4 x 16 bytes at p, p + 32 B, p + 64 B, p + 96 B
ALLIE_DEV void lds_read_f4x4_stride32(const void* p, float4 (&r)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:32\n\tds_read_b128 %2, %4 offset:64\n\t"
      "ds_read_b128 %3, %4 offset:96\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p)
      : "memory");
}
// two 16-byte reads
ALLIE_DEV void lds_read_f4x2(const void* p0, const void* p1, float4& r0, float4& r1) {
  asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(r0), "=&v"(r1)
               : "v"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p0),
                 "v"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p1)
               : "memory");
}
ALLIE_DEV uint32_t lds_off(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
ALLIE_DEV void lds_write_b64(void* p, uint2 v) {
  asm volatile("ds_write_b64 %0, %1" ::"v"(lds_off(p)), "v"(v) : "memory");
}
// four 16-byte reads (untracked, with their wait, as lds_read_f4x2)
ALLIE_DEV void lds_read_b128x4(const void* p0, const void* p1, const void* p2, const void* p3, u32x4_t (&r)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(lds_off(p0)), "v"(lds_off(p1)), "v"(lds_off(p2)), "v"(lds_off(p3))
      : "memory");
}
// An accumulator read where it is used (not all 256 copied out at once
// after the k-loop)
ALLIE_DEV float acc_read(float v) {
  float r;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(v));
  return r;
}

// SCALED: weights that were fp8 (widened exactly to bf16 for this call) with
// a per-output-channel scale: the accumulators start at 0 and the epilogue
// takes acc * scale + bias (the 256x128 kernel's order for fp8 weights).
template <int EPI, bool SCALED, bool KV>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(GemmArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
  // the 256 x 256 geometry (shadows the 256 x 128 kernel's constants)
  constexpr int BM = big::BM, BN = big::BN, BK = big::BK;
  constexpr int FM = big::FM, FN = big::FN, A_STAGE = big::A_STAGE, W_STAGE = big::W_STAGE;
  constexpr int DMA = big::DMA, EP = big::EP;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[big::SMEM];
  auto sA = [&](int s) { return smem + s * A_STAGE; };
  auto sW = [&](int s) { return smem + big::STAGES * A_STAGE + s * W_STAGE; };
  auto bias_lds = [&](int par) { return reinterpret_cast<const float*>(smem + big::BIAS + par * big::SLOT); };
  auto scale_lds = [&](int par) { return reinterpret_cast<const float*>(smem + big::SCALE + par * big::SLOT); };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int num_tm = (a.M + BM - 1) / BM, num_tn = a.N / BN;
  const int tiles = num_tm * num_tn;
  const int K = a.K, KT = K / BK;
  const int wm = wave & 1, wn = wave >> 1;
  const int frow = lane & 31, half = lane >> 5;

  // loader: one DMA instruction fills 8 rows of 128 B (lane -> row lane / 8,
  // physical chunk lane % 8); wave w fills rows [64 w, 64 w + 64) of both
  // the A and the W stage.  Row 64 w + 8 i + lane / 8 holds logical chunk
  // (lane % 8) ^ ((4 i + lane / 16) & 7) in that physical slot.
  const int lc_even = (lane & 7) ^ (lane >> 4);
  // A loads: instruction i reads row 64 w + 8 i + lane / 8 (per-lane offset,
  // so that rows past M fall outside the buffer)
  const uint32_t a_lane = (uint32_t)((wave * 64 + (lane >> 3)) * a.lda * 2);
  const uint32_t a_ev = a_lane + lc_even * 16, a_od = a_lane + (lc_even ^ 4) * 16;

  // W loads: the row group of instruction i goes into the scalar offset
  // (every W row of a tile is valid); two per-lane offsets (even and odd i)
  const uint32_t w_lane = (uint32_t)((lane >> 3) * K * 2);
  const uint32_t w_ev = w_lane + lc_even * 16, w_od = w_lane + (lc_even ^ 4) * 16;

  // per-tile buffers: A over the tile's rows (rows past M read 0), W over
  // its 256 rows, C over its rows (stores past M dropped), the bias slice
  // (without a bias the slice is read from A, always valid, and ignored)
  struct Tile {
    int m0, n0, rows;
  };
  auto make_tile = [&](int t) {
    Tile T;
    int tm, tn;
    tile_coords(t, tiles, num_tm, num_tn, tm, tn);
    T.m0 = tm * BM;
    T.n0 = tn * BN;
    T.rows = a.M - T.m0 < BM ? a.M - T.m0 : BM;
    return T;
  };
  auto rsrc_A = [&](const Tile& T) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(reinterpret_cast<const bf16_t*>(a.A) + (int64_t)T.m0 * a.lda), (short)0,
        T.rows * a.lda * 2, 0x00020000);
  };
  auto rsrc_W = [&](const Tile& T) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(reinterpret_cast<const bf16_t*>(a.W) + (int64_t)T.n0 * K), (short)0, BN * K * 2,
        0x00020000);
  };
  auto rsrc_C = [&](const Tile& T) {
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<bf16_t*>(a.C) + (int64_t)T.m0 * a.ldc, (short)0,
                                             T.rows * a.ldc * 2, 0x00020000);
  };
  auto rsrc_B = [&](const Tile& T) {
    return __builtin_amdgcn_make_buffer_rsrc(
        a.bias ? const_cast<float*>(a.bias + T.n0) : const_cast<void*>(a.A), (short)0, BN * 4, 0x00020000);
  };
  auto rsrc_S = [&](const Tile& T) {
    return __builtin_amdgcn_make_buffer_rsrc(
        (SCALED && a.scale) ? const_cast<float*>(a.scale + T.n0) : const_cast<void*>(a.A), (short)0, BN * 4,
        0x00020000);
  };
  // without a bias the slice lands in the spare slot and the bias slots hold
  // zeros (the load count stays the same either way); likewise the scale
  // slice, which only SCALED reads
  const int bias_dst = opaque_s(a.bias ? big::BIAS : big::SPARE);
  const int scale_dst = opaque_s((SCALED && a.scale) ? big::SCALE : big::SPARE);
  const int slot_step = opaque_s((a.bias ? big::SLOT : 0));
  const int sslot_step = opaque_s(((SCALED && a.scale) ? big::SLOT : 0));
  if (!a.bias) {
    reinterpret_cast<float*>(smem + big::BIAS)[tid] = 0.f;
    reinterpret_cast<float*>(smem + big::BIAS + big::SLOT)[tid] = 0.f;
  }
  // DMA of k-tile kt's A rows (issue_a) or W rows (issue_w) into stage s
  auto issue_a = [&](const Tile& T, int kt, int s) {
    const uint32_t kb = (uint32_t)kt * BK * 2;
    const auto rA = rsrc_A(T);
    bf16_t* la = sA(0) + opaque_s(s * A_STAGE + wave * 64 * BK);
    const uint32_t ae = (uint32_t)opaque_v((int)a_ev), ao = (uint32_t)opaque_v((int)a_od);
    const uint32_t a8 = (uint32_t)opaque_s(8 * a.lda * 2);
#pragma unroll
    for (int i = 0; i < DMA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void_t2*)(la + 8 * i * BK), 16,
                                               ((i & 1) ? ao : ae) + (uint32_t)i * a8, kb, 0, 0);
  };
  auto issue_w = [&](const Tile& T, int kt, int s) {
    const uint32_t kb = (uint32_t)kt * BK * 2;
    const auto rW = rsrc_W(T);
    bf16_t* lw = sW(0) + opaque_s(s * W_STAGE + wave * 64 * BK);
    const uint32_t wk = (uint32_t)opaque_s(wave * 64 * K * 2) + kb;
#pragma unroll
    for (int i = 0; i < DMA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_void_t2*)(lw + 8 * i * BK), 16, (i & 1) ? w_od : w_ev,
                                               wk + (uint32_t)(8 * i * K * 2), 0, 0);
  };
  auto issue = [&](const Tile& T, int kt, int s) {
    issue_a(T, kt, s);
    issue_w(T, kt, s);
  };
  // a tile's head: its bias and scale slices (wave w: 64 values each) into
  // the slots of its parity, and its first two k-tiles
  auto issue_bias = [&](const Tile& T, int par) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_B(T), (lds_void_t2*)(smem + bias_dst + par * slot_step + wave * 128),
                                             4, (uint32_t)(wave * 64 + lane) * 4, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_S(T),
                                             (lds_void_t2*)(smem + scale_dst + par * sslot_step + wave * 128), 4,
                                             (uint32_t)(wave * 64 + lane) * 4, 0, 0, 0);
  };
  auto issue_head = [&](const Tile& T, int par) {
    issue_bias(T, par);
    issue(T, 0, 0);
    issue(T, 1, 1);
  };

  f32x16_t acc[FN][FM];
  // fragment reads: row r = base + frow with base a multiple of 32, so
  // swz(r, c) = base * BK + swz(frow, c); the lane part is recomputed per
  // read group (opaque) rather than kept for every stage and step
  auto load_w = [&](int s, int st, bf16x8_t(&wf)[FN]) {
    const bf16_t* pw = sW(s) + wn * 128 * BK + opaque_v(big::swz(frow, 2 * st + half));
#pragma unroll
    for (int i = 0; i < FN; ++i)
      wf[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(pw + i * 32 * BK));
  };
  auto load_a = [&](int s, int st, bf16x8_t(&xf)[FM]) {
    const bf16_t* pa = sA(s) + wm * 128 * BK + opaque_v(big::swz(frow, 2 * st + half));
#pragma unroll
    for (int j = 0; j < FM; ++j)
      xf[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(pa + j * 32 * BK));
  };
  auto mfma_step = [&](const bf16x8_t(&wf)[FN], const bf16x8_t(&xf)[FM]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
  };
  constexpr int NMF = FN * FM;
  bf16x8_t w0[FN], w1[FN], w2[FN], w3[FN], xP[FM], xQ[FM];

  // One k-tile from stage s.  The W fragments of all four k-steps are read in
  // step 0, so after a barrier the stage's W rows are free and tile kt + 2's
  // W rows load during step 1; after step 2 tile kt + 1 must have landed
  // (`newer` loads issued after it may be in flight) and, past a second
  // barrier, tile kt + 2's A rows load during step 3 while it reads tile
  // kt + 1's first fragments.  Each burst of loads is half a k-tile's, spread
  // between MFMAs (a whole k-tile's loads at one point stall MFMA issue
  // while the texture unit drains them).
  // (RT, rk: the tile and k-tile the refills load -- normally T and kt + 2;
  // hpar >= 0: RT's bias and scale go into slot hpar with its A rows)
  auto k_tile_rf = [&](const Tile& RT, int rk, int hpar, int kt, int newer, auto refill) {
    constexpr bool RF = decltype(refill)::value;
    const int s = kt & 1;
    load_w(s, 1, w1);
    load_w(s, 2, w2);
    load_w(s, 3, w3);
    load_a(s, 1, xQ);
    mfma_step(w0, xP);
    interleave_rwl<16, 0, 0, NMF>();
    lds_barrier();
    if constexpr (RF) issue_w(RT, rk, s);
    load_a(s, 2, xP);
    mfma_step(w1, xQ);
    interleave_rwl<FM, 0, RF ? DMA : 0, NMF>();
    load_a(s, 3, xQ);
    mfma_step(w2, xP);
    interleave_rwl<FM, 0, 0, NMF>();
    switch (newer) {
      case 0: big::wait_vm<0>(); break;
      case DMA: big::wait_vm<DMA>(); break;
      case big::STORES: big::wait_vm<big::STORES>(); break;
      default: big::wait_vm<DMA + big::STORES>(); break;
    }
    lds_barrier();
    if constexpr (RF) {
      if (hpar >= 0) issue_bias(RT, hpar);
      issue_a(RT, rk, s);
    }
    // after the last tile these read a stale (in-bounds) stage, never used
    load_w(s ^ 1, 0, w0);
    load_a(s ^ 1, 0, xP);
    mfma_step(w3, xQ);
    interleave_rwl<FN + FM, 0, RF ? DMA : 0, NMF>();
  };

  auto k_tile = [&](const Tile& T, int kt, int newer, auto refill) { k_tile_rf(T, kt + 2, -1, kt, newer, refill); };

  bf16_t* reg = smem + big::RING + wave * big::CHUNK;
  const int rl = lane >> 3, cl = (lane & 7) * 8;  // read-back: row rl + 8 it, columns cl .. cl + 7
  int t = blockIdx.x;
  Tile cur = make_tile(t);
  int par = 0;  // the current tile's bias / scale slot
  issue_head(cur, par);
  bool first = true;
  while (true) {
    // the tile's bias, scale and k-tile 0 must land (k-tile 1 and the
    // previous tile's stores may still be in flight)
    if (first) big::wait_vm<2 * DMA>();
    else big::wait_vm<2 * DMA + big::STORES>();
    lds_barrier();
    const int n_wave = wn * 128;  // within the tile
    // (the bias slice landed with k-tile 0; read untracked, with its wait in
    // the same statement)
    const float* bl = bias_lds(par) + n_wave + half * 4;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      float4 b[4];
      if constexpr (SCALED) {
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = make_float4(0, 0, 0, 0);
      } else {
        lds_read_f4x4_stride32(bl + i * 32, b);
      }
      f32x16_t init;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        init[q * 4 + 0] = b[q].x;
        init[q * 4 + 1] = b[q].y;
        init[q * 4 + 2] = b[q].z;
        init[q * 4 + 3] = b[q].w;
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = init;
      __builtin_amdgcn_sched_barrier(0);
    }
    load_w(0, 0, w0);
    load_a(0, 0, xP);
    int kt = 0;
    // newer than tile kt + 1: this k-tile's W refill and, in k-tile 0, the
    // previous tile's stores
    const int st0 = first ? 0 : big::STORES;
    const int t_next = t + gridDim.x;
    const bool more = t_next < tiles;
    Tile nxt;
    if (more) nxt = make_tile(t_next);
    // with a next tile (and an even k-tile count, so that its k-tiles 0 and 1
    // land in stages 0 and 1), the last two k-tiles refill their stages with
    // its head, which then loads under them instead of under the epilogue
    const bool early = more && KT >= 4 && (KT & 1) == 0;
    if (KT > 2) k_tile(cur, kt++, DMA + st0, std::true_type{});
    else k_tile(cur, kt++, st0, std::false_type{});
    const int kt_rf = early ? KT : KT - 2;  // k-tiles before this that refill
    for (; kt < kt_rf; ++kt) {
      const bool own = kt + 2 < KT;
      Tile RT;
      RT.m0 = own ? cur.m0 : nxt.m0;
      RT.n0 = own ? cur.n0 : nxt.n0;
      RT.rows = own ? cur.rows : nxt.rows;
      k_tile_rf(RT, own ? kt + 2 : kt + 2 - KT, kt + 2 == KT ? (par ^ 1) : -1, kt, DMA, std::true_type{});
    }
    for (; kt < KT; ++kt) k_tile(cur, kt, 0, std::false_type{});

    // KV: a tile of key / value columns goes to the pool, row by row at the
    // rows' slots.  The slots of this lane's 16 rows load here: without early
    // refill that is before the next tile's head (issued below), so waiting
    // for them does not wait for it; with early refill the head went out in
    // the last two k-tiles, and since loads complete in order the wait for
    // the slots also waits for it (time only, at the KV tiles of a QKV GEMM)
    const int d3 = a.N / 3;
    const bool kv_tile = KV && cur.n0 + big::BN > d3;
    int slot[FM][4];
    if constexpr (KV) {
      if (kv_tile) {
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int m = cur.m0 + wm * 128 + j * 32 + it * 8 + rl;
            slot[j][it] = m < a.M ? a.kv_slot[m] : -1;
          }
      }
    }

    // otherwise the next tile's head loads while this one is written out
    if (more && !early) issue_head(nxt, par ^ 1);

    // ---- epilogue: 8 chunks of 32 rows x 64 columns through LDS -------------
    const auto rC = rsrc_C(cur);
    const int ldc2 = opaque_s(a.ldc * 2);
    const uint32_t c_lane = (uint32_t)((wm * 128 + rl) * ldc2 + (cur.n0 + n_wave + cl) * 2);
    // KV: the layer's slice of the pool; a 64-column chunk is one head's key
    // or value, row m at ((block 2 + kv) H + head) 16 + offset of its slot
    const int Hh = d3 / 64;
    const uint32_t pool_bytes = (uint32_t)a.kv_pool_blocks * 2u * (uint32_t)Hh * 2048u;  // < 4 GiB (host check)
    const auto rP = __builtin_amdgcn_make_buffer_rsrc(
        KV ? reinterpret_cast<bf16_t*>(a.kv_pool) + (int64_t)a.kv_layer * a.kv_pool_blocks * 2 * Hh * 1024
           : reinterpret_cast<bf16_t*>(a.C),
        (short)0, KV ? __builtin_bit_cast(int, pool_bytes) : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < FM; ++j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
          const int i = 2 * h + ii;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v0 = acc_read(acc[i][j][q * 4 + 0]), v1 = acc_read(acc[i][j][q * 4 + 1]);
            float v2 = acc_read(acc[i][j][q * 4 + 2]), v3 = acc_read(acc[i][j][q * 4 + 3]);
            if constexpr (SCALED) {
              const int col = n_wave + i * 32 + q * 8 + half * 4;
              float4 sc, bi;
              lds_read_f4x2(scale_lds(par) + col, bias_lds(par) + col, sc, bi);
              v0 = fmaf(v0, sc.x, bi.x);
              v1 = fmaf(v1, sc.y, bi.y);
              v2 = fmaf(v2, sc.z, bi.z);
              v3 = fmaf(v3, sc.w, bi.w);
            }
            if constexpr (EPI == EPI_GELU) {
              round_bf16x2(v0, v1);
              round_bf16x2(v2, v3);
              v0 = gelu_tanh_fast(v0);
              v1 = gelu_tanh_fast(v1);
              v2 = gelu_tanh_fast(v2);
              v3 = gelu_tanh_fast(v3);
            }
            uint2 p;
            p.x = pack_bf16x2(v0, v1);
            p.y = pack_bf16x2(v2, v3);
            lds_write_b64(reg + frow * EP + ii * 32 + q * 8 + half * 4, p);
          }
        }
        // (LDS operations of one wave run in order: the reads see the writes,
        // and the next chunk's writes come after these reads)
        u32x4_t v[4];
        lds_read_b128x4(reg + rl * EP + cl, reg + (8 + rl) * EP + cl, reg + (16 + rl) * EP + cl,
                        reg + (24 + rl) * EP + cl, v);
        const int c0 = cur.n0 + n_wave + h * 64;  // 64-aligned: q, or one head's key or value
        if (KV && kv_tile && c0 >= d3) {
          const int kvi = c0 >= 2 * d3 ? 1 : 0, head = (c0 - (kvi + 1) * d3) >> 6;
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int sl = slot[j][it];
            const bool ok = sl >= 0 && (sl >> 4) < a.kv_pool_blocks;
            const uint32_t off = ok ? ((((uint32_t)(sl >> 4) * 2u + kvi) * Hh + head) * 16u + (sl & 15)) * 128u + cl * 2
                                    : 0xffffffffu;  // outside the buffer: dropped
            __builtin_amdgcn_raw_buffer_store_b128(v[it], rP, off, 0, 2);
          }
        } else {
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            // row wm 128 + j 32 + it 8 + rl, column n0 + n_wave + h 64 + cl; a
            // non-temporal store (cache policy nt): the output is not read
            // again by this kernel, and kept out of L2 it leaves the A and W
            // panels there (QKV 7%, fc 3% faster)
            __builtin_amdgcn_raw_buffer_store_b128(v[it], rC, c_lane + (uint32_t)((j * 32 + it * 8) * ldc2 + h * 128),
                                                   0, 2);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (!more) break;
    t = t_next;
    cur = nxt;
    par ^= 1;
    first = false;
  }
#endif
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

// Sum of the K splits' partials (in split order) and the epilogue, 4
// consecutive outputs of one row per thread.
template <int EPI, bool FP8, bool F32OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs a) {
  const int n4 = a.N >> 2;
  const int64_t mn4 = (int64_t)a.M * n4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= mn4) return;
  const int m = (int)(idx / n4), n = (int)(idx - (int64_t)m * n4) * 4;
  const float4* p = reinterpret_cast<const float4*>(a.part) + idx;
  float4 v = p[0];
  for (int s = 1; s < a.split; ++s) {
    const float4 t = p[s * mn4];
    v.x += t.x;
    v.y += t.y;
    v.z += t.z;
    v.w += t.w;
  }
  if constexpr (FP8) {
    const float4 sc = *reinterpret_cast<const float4*>(a.scale + n);
    v.x *= sc.x;
    v.y *= sc.y;
    v.z *= sc.z;
    v.w *= sc.w;
  }
  if (a.bias) {
    const float4 b = *reinterpret_cast<const float4*>(a.bias + n);
    v.x += b.x;
    v.y += b.y;
    v.z += b.z;
    v.w += b.w;
  }
  if constexpr (F32OUT) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.C) + (int64_t)m * a.ldc + n) = v;
  } else if constexpr (EPI == EPI_RESID) {
    round_bf16x2(v.x, v.y);
    round_bf16x2(v.z, v.w);
    float4* r = reinterpret_cast<float4*>(a.R + (int64_t)m * a.ldr + n);
    float4 h = *r;
    h.x += v.x;
    h.y += v.y;
    h.z += v.z;
    h.w += v.w;
    *r = h;
  } else {
    if constexpr (EPI == EPI_GELU) {
      round_bf16x2(v.x, v.y);
      round_bf16x2(v.z, v.w);
      v.x = gelu_tanh_fast(v.x);
      v.y = gelu_tanh_fast(v.y);
      v.z = gelu_tanh_fast(v.z);
      v.w = gelu_tanh_fast(v.w);
    }
    uint2 pk;
    pk.x = pack_bf16x2(v.x, v.y);
    pk.y = pack_bf16x2(v.z, v.w);
    *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.C) + (int64_t)m * a.ldc + n) = pk;
  }
}

// The persistent 256 x 256 kernel takes bf16-weight GEMMs with bf16 output
// and a store or gelu epilogue whose 256 x 256 tiles fill every CU at least
// once.
bool use_big(const GemmArgs& a, int wt, bool f32out) {
  // fp8 weights take it when the call brings a bf16 buffer to widen them into
  if ((wt != W_BF16 && !(wt == W_FP8 && a.wdq)) || f32out || a.split > 1 || a.epi == EPI_RESID) return false;
  if (a.N % big::BN != 0 || a.K % big::BK != 0 || a.K < 2 * big::BK) return false;
  // buffer offsets inside a tile are 32-bit
  if ((int64_t)big::BM * a.lda * 2 >= (int64_t)1 << 31 || (int64_t)big::BM * a.ldc * 2 >= (int64_t)1 << 31 ||
      (int64_t)big::BN * a.K * 2 >= (int64_t)1 << 31)
    return false;
  const int64_t tiles = (int64_t)((a.M + big::BM - 1) / big::BM) * (a.N / big::BN);
  return tiles >= 256;
}

// compute units of the current device (the persistent grid)
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// fp8 e4m3 weight bytes -> bf16 (exact; 3 mantissa bits fit in 7), 16 per thread
__global__ __launch_bounds__(256) void widen_fp8_kernel(const uint4* __restrict__ w, uint4* __restrict__ out,
                                                        int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n16) return;
  const uint4 v = w[i];
  const uint32_t b[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o[2 * j] = fp8e4m3_to_bf16(b[j] & 0xffu) | (fp8e4m3_to_bf16((b[j] >> 8) & 0xffu) << 16);
    o[2 * j + 1] = fp8e4m3_to_bf16((b[j] >> 16) & 0xffu) | (fp8e4m3_to_bf16(b[j] >> 24) << 16);
  }
  out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
  out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// Launch of kernel K, timed by events e0 (before) and e1 (after) when given.
template <typename K, typename... Args>
void launch_ev(K kernel, dim3 grid, dim3 block, hipStream_t st, hipEvent_t e0, hipEvent_t e1, Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, st, e0, e1, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, st, args...);
}

// The 128- / 192- / 256-row MFMA kernel (and the split-K reduction), the
// product timed by e0 / e1 when given.
template <int EPI, int WT, bool F32OUT>
void launch_tiles(const GemmArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const int bm = gemm_tile_m(a.M, a.N);
  const int tiles = ((a.M + bm - 1) / bm) * (a.N / BN);
  auto go = [&](auto kernel, int blocks) { launch_ev(kernel, dim3(blocks), dim3(NTHREADS), st, e0, e1, a); };
  constexpr int OUT = F32OUT ? OUT_F32 : OUT_BF16;
  if (a.split > 1) {
    if (bm == 128) go(gemm_mfma_kernel<EPI, WT, OUT_PART, 128>, tiles * a.split);
    else if (bm == 192) go(gemm_mfma_kernel<EPI, WT, OUT_PART, 192>, tiles * a.split);
    else go(gemm_mfma_kernel<EPI, WT, OUT_PART, 256>, tiles * a.split);
    const int64_t n4 = (int64_t)a.M * (a.N / 4);
    hipLaunchKernelGGL((splitk_reduce_kernel<EPI, WT == W_FP8 || WT == W_FP8W, F32OUT>), dim3((unsigned)((n4 + 255) / 256)),
                       dim3(256), 0, st, a);
  } else if (bm == 128) {
    go(gemm_mfma_kernel<EPI, WT, OUT, 128>, tiles);
  } else if (bm == 192) {
    go(gemm_mfma_kernel<EPI, WT, OUT, 192>, tiles);
  } else {
    go(gemm_mfma_kernel<EPI, WT, OUT, 256>, tiles);
  }
}

// Row tiles (of 256) that leave the persistent kernel for the 128-row MFMA
// kernel.  When the persistent kernel's last round of tiles fills at most half
// of the grid, that round costs a whole round for a fraction of the work;
// the rows of its tiles (rounded up to whole row tiles), as 128 x 128 tiles at
// most two per CU, take about half a round (measured: N = 1,024, K = 4,096: a
// 256 x 256 round 103 us, a lone 128 x 128 tile 50 us).
int persistent_peel(int M, int N, int grid) {
  const int m_tiles = (M + big::BM - 1) / big::BM, num_tn = N / big::BN;
  const int64_t T = (int64_t)m_tiles * num_tn;
  const int r = (int)(T % grid);
  if (r == 0 || 2 * r > grid) return 0;
  const int p = (r + num_tn - 1) / num_tn;
  if ((int64_t)(m_tiles - p) * num_tn < 256) return 0;  // the rest must stay persistent
  const int64_t rows = M - (int64_t)(m_tiles - p) * big::BM;
  const int64_t small = ((rows + 127) / 128) * (N / BN);
  return small <= 2 * (int64_t)grid ? p : 0;
}

template <int EPI, int WT, bool F32OUT>
hipError_t launch_mfma(const GemmArgs& a, hipStream_t st) {
  if constexpr (EPI != EPI_RESID) {
    if (use_big(a, WT, F32OUT)) {
      // a multiple of 8 blocks keeps block b on XCD b % 8 in every round
      int grid = device_cus() & ~7;
      grid = grid < 8 ? 8 : grid;
      // rows of a last, mostly empty round of tiles go to the 128-row kernel
      const int peel = persistent_peel(a.M, a.N, grid);
      GemmArgs b = a;  // the persistent part: the first rows
      if (peel) b.M = ((a.M + big::BM - 1) / big::BM - peel) * big::BM;
      const int tiles = ((b.M + big::BM - 1) / big::BM) * (b.N / big::BN);
      grid = tiles < grid ? tiles : grid;
      GemmArgs t = a;  // the rest (bf16 activations and output, the caller's weights)
      t.A = reinterpret_cast<const bf16_t*>(a.A) + (int64_t)b.M * a.lda;
      t.C = reinterpret_cast<bf16_t*>(a.C) + (int64_t)b.M * a.ldc;
      t.M = a.M - b.M;
      t.split = 1;
      if (a.kv_slot) t.kv_slot = a.kv_slot + b.M;
      // a probe times every launch of the product: start with the first, stop
      // with the last
      LaunchProbe* p = launch_probe_take();
      hipEvent_t e0 = p ? p->start : nullptr, e1 = p ? p->stop : nullptr;
      if constexpr (WT == W_FP8) {
        // widen the fp8 weights to bf16 (exact) and scale in the epilogue
        const int64_t n16 = (int64_t)a.N * a.K / 16;
        const dim3 wgrid((unsigned)((n16 + 255) / 256));
        const uint4* w8 = reinterpret_cast<const uint4*>(a.W);
        uint4* w16 = reinterpret_cast<uint4*>(a.wdq);
        b.W = a.wdq;
        launch_ev(widen_fp8_kernel, wgrid, dim3(256), st, e0, nullptr, w8, w16, n16);
        if (EPI == EPI_STORE && a.kv_pool)
          launch_ev(gemm_big_kernel<EPI_STORE, true, true>, dim3(grid), dim3(256), st, nullptr, peel ? nullptr : e1, b);
        else
          launch_ev(gemm_big_kernel<EPI, true, false>, dim3(grid), dim3(256), st, nullptr, peel ? nullptr : e1, b);
      } else {
        if (EPI == EPI_STORE && a.kv_pool)
          launch_ev(gemm_big_kernel<EPI_STORE, false, true>, dim3(grid), dim3(256), st, e0, peel ? nullptr : e1, b);
        else
          launch_ev(gemm_big_kernel<EPI, false, false>, dim3(grid), dim3(256), st, e0, peel ? nullptr : e1, b);
      }
      if (peel) {
        if constexpr (WT == W_FP8) {
          t.W = a.wdq;  // widened above
          launch_tiles<EPI, W_FP8W, F32OUT>(t, st, nullptr, e1);
        } else {
          launch_tiles<EPI, WT, F32OUT>(t, st, nullptr, e1);
        }
      }
      return hipGetLastError();
    }
  }
  LaunchProbe* p = launch_probe_take();
  hipEvent_t e0 = p ? p->start : nullptr, e1 = p ? p->stop : nullptr;
  if constexpr (WT == W_FP8) {
    if (a.wdq) {
      // with a widening buffer: the weights widened to bf16 once, then the
      // bf16 loads (converting fp8 fragments inside the k-loop is about 4x
      // slower: M = 981, N = 5,120, K = 1,280: 117 against 25 us)
      const int64_t n16 = (int64_t)a.N * a.K / 16;
      launch_ev(widen_fp8_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), st, e0, nullptr,
                reinterpret_cast<const uint4*>(a.W), reinterpret_cast<uint4*>(a.wdq), n16);
      GemmArgs b = a;
      b.W = a.wdq;
      launch_tiles<EPI, W_FP8W, F32OUT>(b, st, nullptr, e1);
      return hipGetLastError();
    }
  }
  launch_tiles<EPI, WT, F32OUT>(a, st, e0, e1);
  return hipGetLastError();
}

}  // namespace

namespace allie {

bool gemm_uses_persistent(const GemmArgs& a) {
  return a.M > 0 && (a.epi == EPI_STORE || a.epi == EPI_GELU) && use_big(a, a.wtype, a.out_f32 != 0);
}

bool gemm_stores_kv(const GemmArgs& a) {
  if (!a.kv_pool || !a.kv_slot || a.M <= 0 || a.epi != EPI_STORE || a.out_f32 || a.wtype == W_F32) return false;
  if (a.N % 192 != 0 || a.ldc != a.N) return false;
  if (gemm_skinny_supported(a)) return true;  // the skinny kernel writes C and the pool
  if (a.split > 1 || !gemm_mfma_supported(a)) return false;
  // the persistent kernel addresses one layer's slice with 32-bit offsets
  const bool big = use_big(a, a.wtype, a.out_f32 != 0);
  return !big || (int64_t)a.kv_pool_blocks * 2 * (a.N / 192) * 2048 < ((int64_t)1 << 32);
}

bool gemm_mfma_supported(const GemmArgs& a) {
  return a.N % BN == 0 && a.K % BK == 0 && a.lda % 8 == 0 && a.M > 0;
}

int gemm_tile_m(int M, int N) {
  // 256-row tiles unless that leaves fewer tiles than a 256-CU device has
  // CUs; 192-row ones where they fit one round of 256 and 128-row ones would
  // not (a second, mostly empty round costs as much as a full one).  Kernel
  // trace, weights cold, M = 1,450 (a C4 step): QKV 16.0 against 19.6 us,
  // c_fc 19.9 against 23.7 us; at M = 512 and 4,096 192-row tiles were slower.
  const int64_t tiles256 = (int64_t)((M + 255) / 256) * (N / BN);
  const int64_t tiles192 = (int64_t)((M + 191) / 192) * (N / BN);
  const int64_t tiles128 = (int64_t)((M + 127) / 128) * (N / BN);
  if (tiles128 > 256 && tiles192 <= 256) return 192;
  return tiles256 < 256 ? 128 : 256;
}

int gemm_split_factor(int M, int N, int K) {
  if (M <= 0 || N % BN != 0 || K % BK != 0) return 1;
  const int bm = gemm_tile_m(M, N);
  const int64_t tiles = (int64_t)((M + bm - 1) / bm) * (N / BN);
  const int KT = K / BK;
  int s = 1;
  // double while every split keeps at least 8 k-tiles and the grid stays
  // within a cap: 96 blocks for K < 2048, 256 for longer K.  Measured on the
  // medium model's projections with weights cold in HBM (as in a forward):
  // with few tiles (M <= 256) the extra blocks stream the weights faster
  // (M = 63: K = 1024 at 4 splits 10-11 us against 11.5-15 us unsplit, and
  // K = 4096 at 8 splits 13 us against 44 us); with ~100 tiles (M = 1500) a
  // K = 1024 projection is fastest unsplit (13 us against 18 us at 2
  // splits) while K = 4096 still gains at 2 (32 us against 46 us)
  const int cap = K >= 2048 ? 256 : 96;
  // K = 1024 with at least 32 tiles (the attention c_proj of a C4 half-step,
  // M = 512-750): unsplit 12.1-12.4 us against 12.5-13.8 at the 2 splits the
  // cap allows (allie_gemm_splitk, 24 weight matrices in turn)
  if (K < 2048 && tiles >= 32) return 1;
  while (s < 8 && tiles * s * 2 <= cap && KT % (s * 2) == 0 && KT / (s * 2) >= 8) s *= 2;
  return s;
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t st) {
  if (a.M == 0) return hipSuccess;
  if (a.kv_pool && !gemm_stores_kv(a)) return hipErrorInvalidValue;
  if (a.wtype != W_F32 && gemm_skinny_supported(a)) return launch_gemm_skinny(a, st);
  if (a.ln_h) return hipErrorInvalidValue;  // the LayerNorm prologue exists on the skinny kernel only
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
  if (a.split > 1 && (a.part == nullptr || (a.K / BK) % a.split != 0)) return hipErrorInvalidValue;
  if (a.kv_pool && !gemm_stores_kv(a)) return hipErrorInvalidValue;
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
