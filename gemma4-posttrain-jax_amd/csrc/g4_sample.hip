// Fused next-token sampling over the LM head's output (g4_sample_tokens).
//
// Replaces forward_lm_head's soft-capping (model.py:676-680) followed by _sample_token
// (sampler.py:145-183) for the configurations RL rollouts use (no top-k, no top-p): per row,
//   x      = cast(tanh(l / cap) * cap)            (the capped logits in the activation dtype)
//   token  = argmax(x)                            (temperature <= 0)
//          = argmax(x / T + gumbel)               (otherwise; Gumbel-max = a categorical draw)
//   logp   = x[token] - logsumexp(x)              (full-vocab log-softmax of the unmodified policy)
// in one pass over the row: running max and rescaled sum for the log-softmax, running argmax.
// The Gumbel noise -log(-log(u)) comes from Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel
// random numbers: as easy as 1, 2, 3", SC 2011) keyed by the 64-bit seed, counter = (column/4,
// row, step, 0): reproducible for a fixed seed and independent of the launch shape. `step` may
// live on the device (advanced by the caller between replays of a captured graph).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kSampleThreads = 1024;

struct Philox4 {
  uint32_t v[4];
};

// Philox4x32 with 10 rounds (Salmon et al. 2011, section 5): multipliers 0xD2511F53 /
// 0xCD9E8D57, Weyl key increments 0x9E3779B9 / 0xBB67AE85.
__device__ __forceinline__ Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                                 uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return Philox4{{c0, c1, c2, c3}};
}

// uniform in the open interval (0, 1): 24 random bits, centred in their bucket
__device__ __forceinline__ float uniform01(uint32_t bits) { return ((float)(bits >> 8) + 0.5f) * (1.0f / 16777216.0f); }

struct RowState {
  float m, s;       // running max of x and sum of exp(x - m)
  float best;       // best score so far
  int idx;          // its column
  float best_x;     // x at that column
};

__device__ __forceinline__ void merge(RowState& a, const RowState& b) {
  if (b.m > a.m) {
    a.s = a.s * __expf(a.m - b.m) + b.s;
    a.m = b.m;
  } else if (b.m > kF32Min) {
    a.s += b.s * __expf(b.m - a.m);
  }
  if (b.best > a.best || (b.best == a.best && b.idx < a.idx)) {  // ties: the first column (torch/jax argmax)
    a.best = b.best;
    a.idx = b.idx;
    a.best_x = b.best_x;
  }
}

__device__ __forceinline__ RowState shfl_state(const RowState& x, int mask) {
  RowState y;
  y.m = __shfl_xor(x.m, mask, 64);
  y.s = __shfl_xor(x.s, mask, 64);
  y.best = __shfl_xor(x.best, mask, 64);
  y.idx = __shfl_xor(x.idx, mask, 64);
  y.best_x = __shfl_xor(x.best_x, mask, 64);
  return y;
}

template <bool BF16>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(G4SampleArgs a) {
  using E = Elem<BF16>;
  using T = typename E::T;
  __shared__ RowState red[kSampleThreads / 64];
  const int row = blockIdx.x;
  const T* lrow = reinterpret_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const uint32_t step = a.step ? (uint32_t)*a.step : (uint32_t)a.step_scalar;
  const uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
  const bool greedy = !(a.temperature > 0.f);
  const float cap = a.softcap;  // the reference divides by the cap (no reciprocal)
  RowState st = {kF32Min, 0.f, -INFINITY, 0x7fffffff, 0.f};
  // each thread takes 4 consecutive columns per visit (one Philox block)
  for (int c4 = threadIdx.x; c4 * 4 < a.vocab; c4 += blockDim.x) {
    Philox4 rnd = {{0u, 0u, 0u, 0u}};
    if (!greedy) rnd = philox4x32_10((uint32_t)c4, (uint32_t)row, step, 0u, k0, k1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int colx = 4 * c4 + e;
      if (colx >= a.vocab) break;
      float x = E::load(lrow, colx);
      if (cap > 0.f) x = E::round(tanhf(x / cap) * cap);
      // log-softmax statistics
      if (x > st.m) {
        st.s = st.s * __expf(st.m - x) + 1.f;
        st.m = x;
      } else {
        st.s += __expf(x - st.m);
      }
      float score = x;
      if (!greedy) score = x / a.temperature - __logf(-__logf(uniform01(rnd.v[e])));
      if (score > st.best) {  // columns visited in increasing order per thread: first wins ties
        st.best = score;
        st.idx = colx;
        st.best_x = x;
      }
    }
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) merge(st, shfl_state(st, msk));
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    RowState t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) merge(t, red[i]);
    a.token_out[row] = t.idx;
    a.logp_out[row] = t.best_x - (t.m + __logf(t.s));
  }
}

}  // namespace
}  // namespace g4

extern "C" int g4_sample_tokens(const G4SampleArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_sample_tokens: args is NULL");
  const G4SampleArgs& a = *args;
  if (a.dtype != G4_DTYPE_F32 && a.dtype != G4_DTYPE_BF16)
    return fail(G4_ERR_INVALID, "g4_sample_tokens: dtype %d", a.dtype);
  if (a.batch <= 0 || a.vocab <= 0 || a.row_stride < a.vocab)
    return fail(G4_ERR_INVALID, "g4_sample_tokens: batch %d vocab %d row_stride %lld", a.batch, a.vocab,
                (long long)a.row_stride);
  if (!a.logits || !a.token_out || !a.logp_out) return fail(G4_ERR_INVALID, "g4_sample_tokens: NULL pointer");
  if (!(a.softcap >= 0.f)) return fail(G4_ERR_INVALID, "g4_sample_tokens: softcap must be >= 0");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a.dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(sample_kernel<true>, dim3(a.batch), dim3(kSampleThreads), 0, st, a);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3(a.batch), dim3(kSampleThreads), 0, st, a);
  return check_launch("g4_sample_tokens");
}
