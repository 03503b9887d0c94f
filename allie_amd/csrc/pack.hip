// Ragged packing of game prefixes on the GPU.
//
// Replaces the padding half of UCITokenizer.pad_and_collate
// (reference src/modeling/data.py:281-337): each game keeps its FIRST
// max_len words (data.py:290), the input id is word & 0x3FFF (data.py:320)
// and the position id counts real tokens from 0 (data.py:327).  Instead of a
// right-padded [B, Tmax] batch the result is a flat token stream:
//   cu_seqlens[B+1], ids[T], pos[T], seq_of[T], last_idx[B],
//   blk_off[B+1], block_table[B][max_blocks], slot[T]      (paged KV layout)
// plus the query-tile list of the varlen attention kernel (heaviest tiles
// first).  Two launches: one workgroup scans the lengths, then one workgroup
// per game scatters its tokens.
#include "common.hpp"
#include "kernels.hpp"

namespace {

constexpr int SCAN_THREADS = 1024;

// Block-wide exclusive scan of one int per thread; returns the block total.
__device__ int block_excl_scan(int v, int* sh_wave, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh_wave[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < (SCAN_THREADS / 64) ? sh_wave[lane] : 0;
    int s = w;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      int y = __shfl_up(s, o, 64);
      if (lane >= o) s += y;
    }
    if (lane < SCAN_THREADS / 64) sh_wave[lane] = s - w;  // exclusive wave offsets
    if (lane == SCAN_THREADS / 64 - 1) sh_wave[16] = s;
  }
  __syncthreads();
  int excl = sh_wave[wave] + x - v;
  total = sh_wave[16];
  __syncthreads();
  return excl;
}

__global__ __launch_bounds__(SCAN_THREADS) void pack_scan_kernel(
    const int32_t* __restrict__ lens, int B, int max_len, int block, int q_tile, int capacity,
    int max_blocks,
    int32_t* __restrict__ cu_seqlens, int64_t* __restrict__ in_off,
    int32_t* __restrict__ last_idx, int32_t* __restrict__ blk_off,
    int32_t* __restrict__ tiles, int32_t* __restrict__ status) {
  __shared__ int sh[17];
  int carry_t = 0, carry_b = 0, bad = 0;
  int64_t carry_w = 0;
  int max_tiles = 0;
  for (int base = 0; base < B; base += SCAN_THREADS) {
    int s = base + threadIdx.x;
    int len = s < B ? lens[s] : 0;
    if (s < B && len <= 0) bad |= 1;
    int n = len < max_len ? len : max_len;
    if (n < 0) n = 0;
    int nb = (n + block - 1) / block;
    if (nb > max_blocks) bad |= 4;
    int tot_t, tot_b, tot_w;
    int et = block_excl_scan(n, sh, tot_t);
    int eb = block_excl_scan(nb, sh, tot_b);
    // word offsets can exceed 2^31 only for absurd inputs; scan in 32-bit
    // chunks and widen with the 64-bit carry.
    int ew = block_excl_scan(len > 0 ? len : 0, sh, tot_w);
    if (s < B) {
      cu_seqlens[s] = carry_t + et;
      last_idx[s] = carry_t + et + n - 1;
      blk_off[s] = carry_b + eb;
      in_off[s] = carry_w + ew;
      int nt = (n + q_tile - 1) / q_tile;
      max_tiles = max_tiles > nt ? max_tiles : nt;
    }
    carry_t += tot_t;
    carry_b += tot_b;
    carry_w += tot_w;
  }
  if (threadIdx.x == 0) {
    cu_seqlens[B] = carry_t;
    blk_off[B] = carry_b;
  }
  if (carry_t > capacity) bad |= 2;
  // status is written, not accumulated, so it needs no clearing beforehand
  const int b1 = __syncthreads_or(bad & 1), b4 = __syncthreads_or(bad & 4);
  if (threadIdx.x == 0 && status != nullptr) *status = (b1 ? 1 : 0) | (bad & 2) | (b4 ? 4 : 0);
  if (tiles == nullptr) return;
  // query tiles, heaviest level first: level q holds every game with more
  // than q tiles, in game order.
  max_tiles = (int)wave_max((float)max_tiles);
  __shared__ int sh_max[16];
  if ((threadIdx.x & 63) == 0) sh_max[threadIdx.x >> 6] = max_tiles;
  __syncthreads();
  max_tiles = 0;
  for (int w = 0; w < SCAN_THREADS / 64; ++w) max_tiles = max_tiles > sh_max[w] ? max_tiles : sh_max[w];
  int out = 0;
  for (int q = max_tiles - 1; q >= 0; --q) {
    for (int base = 0; base < B; base += SCAN_THREADS) {
      int s = base + threadIdx.x;
      int n = 0;
      if (s < B) {
        n = lens[s] < max_len ? lens[s] : max_len;
      }
      int pred = (s < B && (n + q_tile - 1) / q_tile > q) ? 1 : 0;
      int tot;
      int e = block_excl_scan(pred, sh, tot);
      if (pred) tiles[out + e] = (s << 5) | q;
      out += tot;
    }
  }
}

__global__ __launch_bounds__(256) void pack_fill_kernel(
    const uint32_t* __restrict__ words, const int32_t* __restrict__ lens, int B, int max_len,
    int block, int first_block, int max_blocks, const int32_t* __restrict__ cu_seqlens,
    const int64_t* __restrict__ in_off, const int32_t* __restrict__ blk_off,
    int32_t* __restrict__ ids, int32_t* __restrict__ pos, int32_t* __restrict__ seq_of,
    int32_t* __restrict__ block_table, int32_t* __restrict__ slot, int capacity, int pad_id,
    int32_t* __restrict__ status, const int32_t* __restrict__ table_in, int max_blocks_in) {
  const int s = blockIdx.x;
  int n = lens[s] < max_len ? lens[s] : max_len;
  if (n < 0) n = 0;
  const int t0 = cu_seqlens[s];
  const int64_t w0 = in_off[s];
  const int b0 = first_block + blk_off[s];
  const int nb = (n + block - 1) / block;
  if (block_table != nullptr)
    for (int j = threadIdx.x; j < max_blocks; j += blockDim.x)
      block_table[(int64_t)s * max_blocks + j] = j < nb ? b0 + j : -1;
  const int n_fit = t0 + n <= capacity ? n : (capacity > t0 ? capacity - t0 : 0);
  int pad_seen = 0;
  for (int j = threadIdx.x; j < n_fit; j += blockDim.x) {
    uint32_t w = words[w0 + j];
    const int32_t id = (int32_t)(w & 0x3FFFu);
    pad_seen |= id == pad_id;
    ids[t0 + j] = id;
    pos[t0 + j] = j;
    seq_of[t0 + j] = s;
    if (slot != nullptr) {
      if (table_in != nullptr) {  // the caller's blocks for this game (-1: no block, not written)
        const int bi = j / block;
        const int b = bi < max_blocks_in ? table_in[(int64_t)s * max_blocks_in + bi] : -1;
        slot[t0 + j] = b >= 0 ? b * block + j % block : -1;
      } else {
        slot[t0 + j] = (b0 + j / block) * block + j % block;
      }
    }
  }
  // a PAD id inside a game would be a masked key in the reference's padded
  // batch (data.py:321) but is an ordinary token here: flag it
  if (__syncthreads_or(pad_seen) && threadIdx.x == 0 && status != nullptr) atomicOr(status, 8);
  // the caller's block table is too short for this game: its tail is not cached
  if (table_in != nullptr && nb > max_blocks_in && threadIdx.x == 0 && status != nullptr) atomicOr(status, 4);
}

}  // namespace

namespace allie {

hipError_t launch_pack(const PackArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, st, a.lens, a.B, a.max_len,
                     a.block, a.q_tile, a.capacity, a.max_blocks, a.cu_seqlens, a.in_off, a.last_idx, a.blk_off, a.tiles,
                     a.status);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.B > 0) {
    hipLaunchKernelGGL(pack_fill_kernel, dim3(a.B), dim3(256), 0, st, a.words, a.lens, a.B,
                       a.max_len, a.block, a.first_block, a.max_blocks, a.cu_seqlens, a.in_off,
                       a.blk_off, a.ids, a.pos, a.seq_of, a.block_table, a.slot, a.capacity,
                       a.pad_id, a.status, a.block_table_in, a.max_blocks_in);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace allie
