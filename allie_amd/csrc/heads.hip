// Policy / value / time heads on the last token of every game.
//
// The heads GEMM (ln_f(h_last) against [wte; w_value; w_time], bias only on
// the two scalar heads) leaves fp32 rows z.  This kernel turns them into
// what the callers read (reference src/evaluation/decode.py:204-226,
// src/modeling/model.py:72-80,105-110):
//   logits = z[0:vocab]                 (tied lm_head, no bias)
//   value  = tanh(z[value_col])         (value head Linear + Tanh)
//   time   = z[time_col]                (time head Linear)
// rounded to bf16 at the points torch autocast rounds them when
// emulate_bf16 is set (logits_raw, when given, receives z before that
// rounding); and, over the move logits 0..n_moves-1 divided by the
// temperature (optionally restricted to a legal-move bitmask):
//   top1 = first index of the maximum (torch.argmax picks the first),
//   max_logit, lse = logsumexp.
// The reference takes the argmax of softmax(logits / T) (decode.py:223-226,
// 112): a NaN or +inf among the considered logits makes that whole softmax
// NaN and torch.argmax then returns its first element, so such a row gets
// top1 = the first considered move id, and max_logit = lse = NaN.
// One workgroup per game.
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace allie;

__global__ __launch_bounds__(256) void heads_kernel(HeadsArgs a) {
  const float temperature = a.temperature;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* z = a.z + (int64_t)b * a.ldz;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  int first_ok = 0x7fffffff;  // first considered move id
  bool nonfinite = false;     // a considered logit / T is NaN or +inf
  for (int c = tid; c < a.vocab; c += 256) {
    float l = z[c];
    if (a.logits_raw) a.logits_raw[(int64_t)b * a.vocab + c] = l;
    if (a.emulate_bf16) l = round_bf16(l);
    if (a.logits) a.logits[(int64_t)b * a.vocab + c] = l;
    if (c < a.n_moves) {
      bool ok = true;
      if (a.legal) ok = (a.legal[(int64_t)b * a.legal_words + (c >> 5)] >> (c & 31)) & 1u;
      if (ok) {
        const float x = l / temperature;
        first_ok = c < first_ok ? c : first_ok;
        if (!(x < INFINITY)) nonfinite = true;  // NaN or +inf
        if (x > best) {  // c increases per thread: keeps the first maximum
          best = x;
          best_i = c;
        }
      }
    }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ float ssum[4];
  __shared__ int sfirst[4];
  nonfinite = __syncthreads_or(nonfinite);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int of = __shfl_xor(first_ok, o, 64);
    first_ok = of < first_ok ? of : first_ok;
  }
  // wave argmax, ties to the lower index
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(best, o, 64);
    int oi = __shfl_xor(best_i, o, 64);
    if (ov > best || (ov == best && oi < best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  const int w = tid >> 6, lane = tid & 63;
  if (lane == 0) {
    sv[w] = best;
    si[w] = best_i;
    sfirst[w] = first_ok;
  }
  __syncthreads();
  best = sv[0];
  best_i = si[0];
  for (int i = 1; i < 4; ++i)
    if (sv[i] > best || (sv[i] == best && si[i] < best_i)) {
      best = sv[i];
      best_i = si[i];
    }
  float s = 0.f;
  if (best > -INFINITY) {
    for (int c = tid; c < a.n_moves; c += 256) {
      bool ok = true;
      if (a.legal) ok = (a.legal[(int64_t)b * a.legal_words + (c >> 5)] >> (c & 31)) & 1u;
      if (ok) {
        float l = z[c];
        if (a.emulate_bf16) l = round_bf16(l);
        s += __expf(l / temperature - best);
      }
    }
  }
  s = wave_sum(s);
  if (lane == 0) ssum[w] = s;
  __syncthreads();
  if (tid == 0) {
    const float tot = (ssum[0] + ssum[1]) + (ssum[2] + ssum[3]);
    if (nonfinite) {
      int f = sfirst[0];
      for (int i = 1; i < 4; ++i) f = sfirst[i] < f ? sfirst[i] : f;
      a.top1[b] = f;
      a.max_logit[b] = NAN;
      a.lse[b] = NAN;
    } else {
      a.top1[b] = best > -INFINITY ? best_i : -1;
      a.max_logit[b] = best;
      a.lse[b] = best > -INFINITY ? best + logf(tot) : -INFINITY;
    }
    float v = z[a.value_col], t = z[a.time_col];
    if (a.emulate_bf16) {
      v = round_bf16(tanhf(round_bf16(v)));
      t = round_bf16(t);
    } else {
      v = tanhf(v);
    }
    a.value[b] = v;
    a.time[b] = t;
  }
}

}  // namespace

namespace allie {

hipError_t launch_heads(const HeadsArgs& a, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  hipLaunchKernelGGL(heads_kernel, dim3(a.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace allie
