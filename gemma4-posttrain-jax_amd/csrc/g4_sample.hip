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

// The soft-capped logit of column col (cap 0: the logit itself); bf16 logits go through the table.
template <bool BF16>
__device__ __forceinline__ float capped_at(const typename Elem<BF16>::T* row, int col, const CapTable& t) {
  using E = Elem<BF16>;
  if (!(t.cap > 0.f)) return E::load(row, col);
  if constexpr (BF16) return capped(reinterpret_cast<const uint16_t*>(row)[col], t);
  else return E::round(tanhf(E::load(row, col) / t.cap) * t.cap);  // the reference divides by the cap
}

template <bool BF16, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(G4SampleArgs a) {
  using T = typename Elem<BF16>::T;
  __shared__ RowState red[kSampleThreads / 64];
  __shared__ uint16_t cap_tab[BF16 ? kCapTableEntries : 1];
  const int row = blockIdx.x;
  const CapTable ct = cap_table(cap_tab, a.softcap);
  if (BF16 && a.softcap > 0.f) {
    cap_table_fill(cap_tab, a.softcap, threadIdx.x, kSampleThreads);
    __syncthreads();
  }
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
    if (mx > st.m) {  // a new running max: rescale the sum (else the factor would be exactly 1)
      st.s *= expf(st.m - mx);
      st.m = mx;
    }
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < N; ++u) sum += expf(x[u] - st.m);
    st.s += sum;
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
      if (takes_best(score[u], st.best)) {
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
        if constexpr (BF16) {
          const uint32_t bits = e & 1 ? word >> 16 : word & 0xffffu;
          x[e] = a.softcap > 0.f ? capped(bits, ct) : bf16_bits_to_f32(bits);
        } else {
          x[e] = __uint_as_float(word);
          if (a.softcap > 0.f) x[e] = E::round(tanhf(x[e] / a.softcap) * a.softcap);  // the reference divides by the cap
        }
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
        x[u] = c < a.vocab ? capped_at<BF16>(lrow, c, ct) : -INFINITY;
      }
      step(x, c0, kSampleThreads);
    }
  }
  if (proposal) {
    const float* prow = a.proposal + (int64_t)row * a.proposal_width;
    for (int j = threadIdx.x; j < a.proposal_width; j += kSampleThreads) {
      const float score = prow[j] + gumbel(k0, k1, (uint64_t)row * (uint64_t)a.proposal_width + (uint64_t)j);
      if (takes_best(score, st.best)) {
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
    // only a row whose every score is -inf keeps no best: clamp so that every read below stays in bounds
    const int width = proposal ? a.proposal_width : a.vocab;
    int token = t.idx < 0 ? 0 : (t.idx >= width ? width - 1 : t.idx);
    if (proposal && a.proposal_index) token = a.proposal_index[(int64_t)row * a.proposal_width + token];
    token = token < 0 ? 0 : (token >= a.vocab ? a.vocab - 1 : token);
    const float x = capped_at<BF16>(lrow, token, ct);
    a.token_out[row] = token;
    a.logp_out[row] = (x - t.m) - logf(t.s);
  }
}

// out = bf16(tanh(x / cap) * cap) elementwise over bf16 x, through the soft-cap table (each
// workgroup fills its own); 8 elements per thread and step with 16-byte accesses, then the tail.
constexpr int kCapThreads = 256;

__global__ __launch_bounds__(kCapThreads) void softcap_kernel(const uint16_t* x, uint16_t* out, int64_t n, float cap) {
  __shared__ uint16_t tab[kCapTableEntries];
  cap_table_fill(tab, cap, threadIdx.x, kCapThreads);
  __syncthreads();
  const CapTable ct = cap_table(tab, cap);
  const int64_t n8 = n / 8;
  const int64_t stride = (int64_t)gridDim.x * kCapThreads;
  for (int64_t i = (int64_t)blockIdx.x * kCapThreads + threadIdx.x; i < n8; i += stride) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + 8 * i);
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = f32_to_bf16_bits(capped(w[q] & 0xffffu, ct)) | (f32_to_bf16_bits(capped(w[q] >> 16, ct)) << 16);
    *reinterpret_cast<u32x4*>(out + 8 * i) = o;
  }
  for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * kCapThreads + threadIdx.x; i < n; i += stride)
    out[i] = (uint16_t)f32_to_bf16_bits(capped(x[i], ct));
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

extern "C" int g4_softcap_bf16(int64_t n, const void* x, float cap, void* out, void* stream) {
  using namespace g4;
  if (n < 0) return fail(G4_ERR_INVALID, "g4_softcap_bf16: n %lld", (long long)n);
  if (!(cap > 0.f) || !(cap < INFINITY)) return fail(G4_ERR_INVALID, "g4_softcap_bf16: cap must be finite and > 0");
  if (n == 0) return G4_OK;
  if (!x || !out) return fail(G4_ERR_INVALID, "g4_softcap_bf16: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(out) & 15))
    return fail(G4_ERR_INVALID, "g4_softcap_bf16: x and out need 16-byte alignment");
  const int64_t want = (n / 8 + kCapThreads - 1) / kCapThreads;
  const unsigned grid = (unsigned)(want < 1 ? 1 : (want > 1024 ? 1024 : want));
  hipLaunchKernelGGL(softcap_kernel, dim3(grid), dim3(kCapThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), n, cap);
  return check_launch("g4_softcap_bf16");
}
