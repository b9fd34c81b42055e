// Fused next-token sampling over the LM head's output (g4_sample_tokens).
//
// One step of generate's loop body (sampler.py:265-270): split the generation key, then
// _sample_token (sampler.py:145-183) on the soft-capped logits (model.py:676-680), in one pass
// over each row: running max / rescaled sum for the full-vocab log-softmax and a running
// argmax of the perturbed scores. The random stream is JAX's: threefry2x32 (Salmon, Moraes, Dror,
// Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011; 20 rounds, the Skein rotation
// constants), key splitting and random bits in JAX's partitionable layout, uniform floats from
// the top 23 bits, Gumbel noise -log(-log(u)) and categorical = argmax(scores + noise).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kSampleThreads = 1024;
#include "g4_sample_common.h"  // threefry2x32, Gumbel noise, the per-row running state

template <bool BF16>
__device__ __forceinline__ float capped(const typename Elem<BF16>::T* row, int col, float cap) {
  using E = Elem<BF16>;
  float x = E::load(row, col);
  if (cap > 0.f) x = E::round(tanhf(x / cap) * cap);  // the reference divides by the cap
  return x;
}

template <bool BF16, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(G4SampleArgs a) {
  using T = typename Elem<BF16>::T;
  __shared__ RowState red[kSampleThreads / 64];
  const int row = blockIdx.x;
  const T* lrow = reinterpret_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const bool greedy = !(a.temperature > 0.f);
  const bool proposal = !greedy && a.proposal != nullptr;
  uint32_t k0 = 0u, k1 = 0u;
  if (!greedy) {
    if (a.split_key) {  // sample_key = split(key)[1] = threefry2x32(key, (0, 1))
      k0 = 0u;
      k1 = 1u;
      threefry2x32(a.key[0], a.key[1], k0, k1);
    } else {
      k0 = a.key[0];
      k1 = a.key[1];
    }
  }
  RowState st = {kF32Min, 0.f, -INFINITY, 0x7fffffff};
  // One step over N columns col0 + u * stride (u = 0 .. N-1, increasing): the max / sum rescale once
  // per step, then the perturbed scores (N independent noise chains). Each thread visits its columns
  // in increasing order, so a strict comparison keeps the first of equal scores.
  auto step = [&](auto& x, int col0, int stride) {
    constexpr int N = sizeof(x) / sizeof(x[0]);
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < N; ++u) mx = fmaxf(mx, x[u]);
    const float mn = fmaxf(st.m, mx);
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < N; ++u) sum += expf(x[u] - mn);
    st.s = st.s * expf(st.m - mn) + sum;
    st.m = mn;
    if (proposal) return;
    float score[N];
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int c = col0 + u * stride;
      score[u] = x[u];
      if (!greedy && c < a.vocab) {
        const float t = a.temperature == 1.0f ? x[u] : x[u] / a.temperature;
        score[u] = t + gumbel(k0, k1, (uint64_t)row * (uint64_t)a.vocab + (uint64_t)c);
      }
    }
#pragma unroll
    for (int u = 0; u < N; ++u) {
      if (score[u] > st.best) {
        st.best = score[u];
        st.idx = col0 + u * stride;
      }
    }
  };
  if (VEC) {
    // 8 consecutive columns per thread and step (one 16-byte bf16 load, two for f32), the next
    // step's columns requested before this step's arithmetic.
    using E = Elem<BF16>;
    constexpr int kRaw = BF16 ? 1 : 2;
    const int nchunks = a.vocab / 8;
    u32x4 cur[kRaw], nxt[kRaw];
    auto load_raw = [&](int j, u32x4 (&r)[kRaw]) {
#pragma unroll
      for (int q = 0; q < kRaw; ++q) r[q] = *reinterpret_cast<const u32x4*>(lrow + 8 * j + 4 * q * (BF16 ? 2 : 1));
    };
    int j = threadIdx.x;
    if (j < nchunks) load_raw(j, nxt);
    for (; j < nchunks; j += kSampleThreads) {
#pragma unroll
      for (int q = 0; q < kRaw; ++q) cur[q] = nxt[q];
      if (j + kSampleThreads < nchunks) load_raw(j + kSampleThreads, nxt);
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = cur[BF16 ? 0 : e / 4][BF16 ? e / 2 : e % 4];
        x[e] = BF16 ? (e & 1 ? __uint_as_float(word & 0xffff0000u) : __uint_as_float(word << 16)) : __uint_as_float(word);
        if (a.softcap > 0.f) x[e] = E::round(tanhf(x[e] / a.softcap) * a.softcap);  // the reference divides by the cap
      }
      step(x, 8 * j, 1);
    }
  } else {
    // columns c = tid + 1024 (4 n + u)
    constexpr int kUnroll = 4;
    for (int c0 = threadIdx.x; c0 < a.vocab; c0 += kUnroll * kSampleThreads) {
      float x[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = c0 + u * kSampleThreads;
        x[u] = c < a.vocab ? capped<BF16>(lrow, c, a.softcap) : -INFINITY;
      }
      step(x, c0, kSampleThreads);
    }
  }
  if (proposal) {
    const float* prow = a.proposal + (int64_t)row * a.proposal_width;
    for (int j = threadIdx.x; j < a.proposal_width; j += kSampleThreads) {
      const float score = prow[j] + gumbel(k0, k1, (uint64_t)row * (uint64_t)a.proposal_width + (uint64_t)j);
      if (score > st.best) {
        st.best = score;
        st.idx = j;
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
    for (int i = 1; i < kSampleThreads / 64; ++i) merge(t, red[i]);
    // a row of NaN scores keeps no best: clamp so that every read below stays in bounds
    const int width = proposal ? a.proposal_width : a.vocab;
    int token = t.idx < 0 ? 0 : (t.idx >= width ? width - 1 : t.idx);
    if (proposal && a.proposal_index) token = a.proposal_index[(int64_t)row * a.proposal_width + token];
    token = token < 0 ? 0 : (token >= a.vocab ? a.vocab - 1 : token);
    const float x = capped<BF16>(lrow, token, a.softcap);
    a.token_out[row] = token;
    a.logp_out[row] = (x - t.m) - logf(t.s);
  }
}

// key <- split(key)[0] = threefry2x32(key, (0, 0)), after every row has read the old key
__global__ void advance_key_kernel(uint32_t* key) {
  if (threadIdx.x == 0) {
    uint32_t x0 = 0u, x1 = 0u;
    threefry2x32(key[0], key[1], x0, x1);
    key[0] = x0;
    key[1] = x1;
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
  const bool greedy = !(a.temperature > 0.f);
  if (!greedy && !a.key) return fail(G4_ERR_INVALID, "g4_sample_tokens: sampling needs the device key");
  if (a.split_key != 0 && a.split_key != 1) return fail(G4_ERR_INVALID, "g4_sample_tokens: split_key %d", a.split_key);
  if (a.proposal) {
    if (a.proposal_width <= 0) return fail(G4_ERR_INVALID, "g4_sample_tokens: proposal_width %d", a.proposal_width);
    if (!a.proposal_index && a.proposal_width > a.vocab)
      return fail(G4_ERR_INVALID, "g4_sample_tokens: proposal_width %d > vocab %d without proposal_index",
                  a.proposal_width, a.vocab);
  } else if (a.proposal_width != 0 || a.proposal_index) {
    return fail(G4_ERR_INVALID, "g4_sample_tokens: proposal_width / proposal_index without a proposal");
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t esize = a.dtype == G4_DTYPE_BF16 ? 2 : 4;
  const bool vec = a.vocab % 8 == 0 && (a.row_stride * esize) % 16 == 0 && reinterpret_cast<uintptr_t>(a.logits) % 16 == 0;
  if (a.dtype == G4_DTYPE_BF16) {
    if (vec)
      hipLaunchKernelGGL((sample_kernel<true, true>), dim3(a.batch), dim3(kSampleThreads), 0, st, a);
    else
      hipLaunchKernelGGL((sample_kernel<true, false>), dim3(a.batch), dim3(kSampleThreads), 0, st, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((sample_kernel<false, true>), dim3(a.batch), dim3(kSampleThreads), 0, st, a);
    else
      hipLaunchKernelGGL((sample_kernel<false, false>), dim3(a.batch), dim3(kSampleThreads), 0, st, a);
  }
  if (int rc = check_launch("g4_sample_tokens")) return rc;
  if (a.key && a.split_key) {
    hipLaunchKernelGGL(advance_key_kernel, dim3(1), dim3(64), 0, st, a.key);
    return check_launch("g4_sample_tokens (key split)");
  }
  return G4_OK;
}
