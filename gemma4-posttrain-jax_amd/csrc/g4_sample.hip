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

// ---- top-k (+ top-p) draw: the truncated branch of _sample_token (sampler.py:162-183) ----------------
//
// One 1024-thread workgroup per row. Scores s = capped logit / T are ranked by an order-preserving
// 32-bit key (ties: the lower vocab id first, as lax.top_k and the oracle's stable argsort do;
// -0.0 counts as +0.0).
// 1. One pass over the row: the full-vocab log-softmax state (max, sum) of the capped logits and
//    each thread's four largest keys. The k-th largest of those 4096 keys, found by a radix select
//    in LDS, is a lower bound L of the row's k-th largest key.
// 2. A second pass gathers every element with key >= L (at least k of them; for random logits a
//    few more than k) into LDS; each candidate's rank among them is its count of larger (key, -id)
//    pairs, and ranks below k give the sorted proposal. Should more than kTkCand elements reach L
//    (heavy ties at the top), the exact threshold t is searched instead (a count per candidate key
//    value), the elements above it are gathered, and the lowest-id elements equal to t follow in
//    id order (thread-contiguous id ranges and a block scan).
// 3. top-p over the k proposal scores (sampler.py:170-178: exp against the first, the normalizing
//    sum in the oracle's pairwise order, the mass before each column from the sequential cumulative
//    sum, the first column always kept), then categorical over the k columns: Gumbel noise of
//    column j at flat index row * k + j of the sample key, the first largest perturbed score wins.
// The log-probability is the full policy's at the drawn id; the loop key is split afterwards by
// advance_key_kernel.
constexpr int kTkMaxK = 256;
constexpr int kTkCand = 2048;

__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s == 0.f ? 0.f : s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_score(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// numpy's float32 pairwise summation (the oracle's w.sum), for n <= 256: runs of at most 128
// elements summed with 8 interleaved partial sums (fewer than 8: in order), a longer run split at
// its 8-aligned half
__device__ __forceinline__ float pairwise_block_f32(const float* a, int n) {
  if (n < 8) {
    float r = 0.f;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  int i = 8;
  for (; i < n - (n % 8); i += 8)
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] += a[i + j];
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}

__device__ __forceinline__ int pairwise_half(int n) { return n / 2 - (n / 2) % 8; }

__device__ __forceinline__ float pairwise_sum_f32(const float* a, int n) {
  if (n <= 128) return pairwise_block_f32(a, n);
  const int n2 = pairwise_half(n);  // <= 128 for n <= 256
  const int m = n - n2;
  float right;
  if (m <= 128) {
    right = pairwise_block_f32(a + n2, m);
  } else {
    const int m2 = pairwise_half(m);
    right = pairwise_block_f32(a + n2, m2) + pairwise_block_f32(a + n2 + m2, m - m2);
  }
  return pairwise_block_f32(a, n2) + right;
}

template <bool BF16, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_top_k_kernel(G4SampleTopKArgs a) {
  using T = typename Elem<BF16>::T;
  __shared__ uint16_t cap_tab[BF16 ? kCapTableEntries : 1];
  __shared__ uint32_t tk4[4 * kSampleThreads];  // each thread's four largest keys
  __shared__ uint32_t hist[256];
  __shared__ uint32_t cand_key[kTkCand];
  __shared__ int32_t cand_id[kTkCand];
  __shared__ float cand_x[kTkCand];
  __shared__ float prop_s[kTkMaxK];
  __shared__ int32_t prop_id[kTkMaxK];
  __shared__ float prop_x[kTkMaxK];
  __shared__ RowState red[kSampleThreads / 64];
  __shared__ uint32_t scan[kSampleThreads];
  __shared__ uint32_t s_count, s_bin, s_need;
  __shared__ float s_best[kSampleThreads / 64];
  __shared__ int s_best_j[kSampleThreads / 64];

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int V = a.vocab, K = a.top_k;
  const CapTable ct = cap_table(cap_tab, a.softcap);
  if (BF16 && a.softcap > 0.f) {
    cap_table_fill(cap_tab, a.softcap, tid, kSampleThreads);
    __syncthreads();
  }
  const T* lrow = reinterpret_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const bool unit_t = a.temperature == 1.0f;
  auto capped_x = [&](int c) { return capped_at<BF16>(lrow, c, ct); };
  auto key_of = [&](float x) { return score_key(unit_t ? x : x / a.temperature); };

  // The columns a thread owns: VEC, 8 consecutive columns per 16-byte (bf16) or 2 x 16-byte (f32)
  // load, chunks j = tid, tid + 1024, ...; otherwise columns tid, tid + 1024, ...
  const int nchunks = a.vocab / 8;
  auto load_x8 = [&](int jj, float (&x)[8]) {
    using E = Elem<BF16>;
    constexpr int kRaw = BF16 ? 1 : 2;
    u32x4 r[kRaw];
#pragma unroll
    for (int q = 0; q < kRaw; ++q) r[q] = *reinterpret_cast<const u32x4*>(lrow + 8 * jj + 4 * q * (BF16 ? 2 : 1));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t word = r[BF16 ? 0 : e / 4][BF16 ? e / 2 : e % 4];
      if constexpr (BF16) {
        const uint32_t bits = e & 1 ? word >> 16 : word & 0xffffu;
        x[e] = a.softcap > 0.f ? capped(bits, ct) : bf16_bits_to_f32(bits);
      } else {
        x[e] = __uint_as_float(word);
        if (a.softcap > 0.f) x[e] = E::round(tanhf(x[e] / a.softcap) * a.softcap);  // the reference divides by the cap
      }
    }
  };

  // ---- pass 1: log-softmax state and each thread's four largest keys (with their columns) ----------
  RowState st = {kF32Min, 0.f, -INFINITY, 0x7fffffff};
  uint32_t t0 = 0u, t1 = 0u, t2 = 0u, t3 = 0u;  // key 0 is no element (every score's key is above it)
  int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
  auto keep = [&](uint32_t k, int c) {  // the four largest keys, the earlier column first among equal ones
    if (k > t3) {
      t3 = k;
      i3 = c;
      if (t3 > t2) { const uint32_t t = t2; t2 = t3; t3 = t; const int ic = i2; i2 = i3; i3 = ic; }
      if (t2 > t1) { const uint32_t t = t1; t1 = t2; t2 = t; const int ic = i1; i1 = i2; i2 = ic; }
      if (t1 > t0) { const uint32_t t = t0; t0 = t1; t1 = t; const int ic = i0; i0 = i1; i1 = ic; }
    }
  };
  auto add_state = [&](const float* x, int n) {
    float mx = x[0];
    for (int u = 1; u < n; ++u) mx = fmaxf(mx, x[u]);
    if (mx > st.m) {
      st.s *= expf(st.m - mx);
      st.m = mx;
    }
    for (int u = 0; u < n; ++u) st.s += expf(x[u] - st.m);
  };
  if constexpr (VEC) {
    for (int jj = tid; jj < nchunks; jj += kSampleThreads) {
      float x[8];
      load_x8(jj, x);
      add_state(x, 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) keep(key_of(x[e]), 8 * jj + e);
    }
  } else {
    for (int c0 = tid; c0 < V; c0 += 4 * kSampleThreads) {
      float x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = c0 + u * kSampleThreads;
        x[u] = c < V ? capped_x(c) : -INFINITY;
      }
      add_state(x, 4);  // the -inf of a column past the row adds exp(-inf) = 0
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (c0 + u * kSampleThreads < V) keep(key_of(x[u]), c0 + u * kSampleThreads);
    }
  }
  tk4[4 * tid] = t0;
  tk4[4 * tid + 1] = t1;
  tk4[4 * tid + 2] = t2;
  tk4[4 * tid + 3] = t3;
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) merge(st, shfl_state(st, msk));
  if (lane == 0) red[wv] = st;
  __syncthreads();
  RowState full = red[0];
  for (int i = 1; i < kSampleThreads / 64; ++i) merge(full, red[i]);

  // radix select over the keys in `src` (n of them, all in LDS): the need-th largest (need >= 1)
  auto select_kth = [&](const uint32_t* src, int n, int need) -> uint32_t {
    uint32_t prefix = 0u;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0u;
      __syncthreads();
      for (int i = tid; i < n; i += kSampleThreads) {
        const uint32_t k = src[i];
        if (shift == 24 || (k >> (shift + 8)) == (prefix >> (shift + 8))) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0u;
        int bin = 255;
        for (; bin > 0; --bin) {
          if (cum + hist[bin] >= (uint32_t)need) break;
          cum += hist[bin];
        }
        s_bin = (uint32_t)bin;
        s_need = (uint32_t)need - cum;
      }
      __syncthreads();
      prefix |= s_bin << shift;
      need = (int)s_need;
      __syncthreads();
    }
    return prefix;
  };
  // the K-th largest of the 4096 kept keys: <= the row's K-th largest key, and >= 1 (the kept keys
  // hold at least min(4096, V) > K real ones)
  const uint32_t lower = select_kth(tk4, 4 * kSampleThreads, K);

  // ---- pass 2: candidates with key >= lower ------------------------------------------------------
  // A thread whose fourth kept key is below `lower` has every such element among its first three
  // kept ones (any other is at most its fourth key); only a thread whose fourth kept key reaches
  // `lower` may hold more, and rescans its columns. For a row without heavy ties at the top that is
  // almost no thread, so the row is read about once.
  auto gather = [&](int c, float x, uint32_t k, bool take) {
    const uint64_t m = __ballot(take);
    if (m == 0ull) return;
    uint32_t base = 0u;
    if (lane == __ffsll((long long)m) - 1) base = atomicAdd(&s_count, (uint32_t)__popcll(m));
    base = __shfl(base, __ffsll((long long)m) - 1, 64);
    if (take) {
      const uint32_t pos = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
      if (pos < (uint32_t)kTkCand) {
        cand_key[pos] = k;
        cand_id[pos] = c;
        cand_x[pos] = x;
      }
    }
  };
  if (tid == 0) s_count = 0u;
  __syncthreads();
  const bool rescan = t3 >= lower;
  {
    const uint32_t tk[3] = {t0, t1, t2};
    const int ik[3] = {i0, i1, i2};
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const bool take = !rescan && tk[q] >= lower;
      gather(ik[q], take ? capped_x(ik[q]) : 0.f, tk[q], take);
    }
  }
  if (__ballot(rescan) != 0ull) {  // whole waves iterate together (ballots)
    if constexpr (VEC) {
      for (int jj = tid; jj - lane < nchunks; jj += kSampleThreads) {
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const bool live = rescan && jj < nchunks;
        if (live) load_x8(jj, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t k = live ? key_of(x[e]) : 0u;
          gather(8 * jj + e, x[e], k, live && k >= lower);
        }
      }
    } else {
      for (int c = tid; c - lane < V; c += kSampleThreads) {
        float x = 0.f;
        uint32_t k = 0u;
        const bool live = rescan && c < V;
        if (live) {
          x = capped_x(c);
          k = key_of(x);
        }
        gather(c, x, k, live && k >= lower);
      }
    }
  }
  __syncthreads();
  uint32_t n_cand = s_count;
  if (n_cand > (uint32_t)kTkCand) {
    // heavy ties at the top: the exact K-th largest key t is the largest value v with
    // count(key >= v) >= K, set bit by bit from the top (one count pass per bit)
    uint32_t thr = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t trial = thr | (1u << bit);
      if (trial <= thr) continue;
      uint32_t cnt = 0u;
      for (int c = tid; c < V; c += kSampleThreads) cnt += key_of(capped_x(c)) >= trial;
      cnt = (uint32_t)__reduce_add_sync(~0ull, cnt);
      if (lane == 0) scan[wv] = cnt;
      __syncthreads();
      uint32_t total = 0u;
      for (int i = 0; i < kSampleThreads / 64; ++i) total += scan[i];
      __syncthreads();
      if (total >= (uint32_t)K) thr = trial;
    }
    // the elements above thr (fewer than K), then the lowest ids equal to thr in id order
    if (tid == 0) s_count = 0u;
    __syncthreads();
    for (int c = tid; c - lane < V; c += kSampleThreads) {
      float x = 0.f;
      uint32_t k = 0u;
      if (c < V) {
        x = capped_x(c);
        k = key_of(x);
      }
      gather(c, x, k, c < V && k > thr);
    }
    __syncthreads();
    const uint32_t n_gt = s_count;
    const int per = (V + kSampleThreads - 1) / kSampleThreads;  // thread-contiguous id ranges
    const int lo = tid * per, hi = min(V, lo + per);
    uint32_t mine = 0u;
    for (int c = lo; c < hi; ++c) mine += key_of(capped_x(c)) == thr;
    scan[tid] = mine;
    __syncthreads();
    for (int off = 1; off < kSampleThreads; off <<= 1) {  // inclusive scan (Hillis-Steele)
      const uint32_t v = tid >= off ? scan[tid - off] : 0u;
      __syncthreads();
      scan[tid] += v;
      __syncthreads();
    }
    uint32_t pos = n_gt + scan[tid] - mine;
    for (int c = lo; c < hi && pos < (uint32_t)K; ++c) {
      const float x = capped_x(c);
      if (key_of(x) == thr) {
        cand_key[pos] = thr;
        cand_id[pos] = c;
        cand_x[pos] = x;
        ++pos;
      }
    }
    __syncthreads();
    n_cand = (uint32_t)K;
  }

  // ---- the sorted proposal: rank of each candidate among them ------------------------------------
  for (int e = tid; e < (int)n_cand; e += kSampleThreads) {
    const uint32_t ke = cand_key[e];
    const int ie = cand_id[e];
    int r = 0;
    for (int j = 0; j < (int)n_cand; ++j) {
      const uint32_t kj = cand_key[j];
      r += (kj > ke) || (kj == ke && cand_id[j] < ie);
    }
    if (r < K) {
      prop_s[r] = key_score(ke);
      prop_id[r] = ie;
      prop_x[r] = cand_x[e];
    }
  }
  __syncthreads();

  // ---- top-p over the proposal --------------------------------------------------------------------
  if (a.top_p < 1.f) {
    float* w = reinterpret_cast<float*>(cand_x);  // reused: the candidates are in the proposal now
    if (tid < K) w[tid] = expf(prop_s[tid] - prop_s[0]);
    __syncthreads();
    if (tid == 0) {
      const float total = pairwise_sum_f32(w, K);
      float cum = 0.f;
      for (int j = 0; j < K; ++j) {
        const float prob = w[j] / total;
        if (j > 0 && !(cum < a.top_p)) prop_s[j] = -INFINITY;  // the mass before column j
        cum += prob;
      }
    }
    __syncthreads();
  }

  // ---- categorical over the K columns ------------------------------------------------------------
  uint32_t k0 = a.key[0], k1 = a.key[1];
  if (a.split_key) {  // sample_key = split(key)[1] = threefry2x32(key, (0, 1))
    uint32_t x0 = 0u, x1 = 1u;
    threefry2x32(k0, k1, x0, x1);
    k0 = x0;
    k1 = x1;
  }
  float best = -INFINITY;
  int best_j = 0x7fffffff;
  if (tid < K) {
    best = prop_s[tid] + gumbel(k0, k1, (uint64_t)row * (uint64_t)K + (uint64_t)tid);
    best_j = tid;
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    const float ob = __shfl_xor(best, msk, 64);
    const int oj = __shfl_xor(best_j, msk, 64);
    if (beats(ob, oj, best, best_j)) {
      best = ob;
      best_j = oj;
    }
  }
  if (lane == 0) {
    s_best[wv] = best;
    s_best_j[wv] = best_j;
  }
  __syncthreads();
  if (tid == 0) {
    float b = s_best[0];
    int j = s_best_j[0];
    for (int i = 1; i < (K + 63) / 64; ++i)
      if (beats(s_best[i], s_best_j[i], b, j)) {
        b = s_best[i];
        j = s_best_j[i];
      }
    j = j < 0 ? 0 : (j >= K ? K - 1 : j);
    a.token_out[row] = prop_id[j];
    a.logp_out[row] = (prop_x[j] - full.m) - logf(full.s);
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

extern "C" int g4_sample_top_k(const G4SampleTopKArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_sample_top_k: args is NULL");
  const G4SampleTopKArgs& a = *args;
  if (a.dtype != G4_DTYPE_F32 && a.dtype != G4_DTYPE_BF16) return fail(G4_ERR_INVALID, "g4_sample_top_k: dtype %d", a.dtype);
  if (a.batch <= 0 || a.vocab <= 0 || a.row_stride < a.vocab)
    return fail(G4_ERR_INVALID, "g4_sample_top_k: batch %d vocab %d row_stride %lld", a.batch, a.vocab,
                (long long)a.row_stride);
  if (a.top_k <= 0 || a.top_k >= a.vocab || a.top_k > kTkMaxK)
    return fail(G4_ERR_UNSUPPORTED, "g4_sample_top_k: top_k %d (1..%d and below the vocab %d)", a.top_k, kTkMaxK,
                a.vocab);
  if (!(a.temperature > 0.f) || !(a.temperature < INFINITY))
    return fail(G4_ERR_INVALID, "g4_sample_top_k: temperature must be finite and > 0 (greedy takes the argmax)");
  if (!(a.top_p > 0.f && a.top_p <= 1.f)) return fail(G4_ERR_INVALID, "g4_sample_top_k: top_p must be in (0, 1]");
  if (!(a.softcap >= 0.f)) return fail(G4_ERR_INVALID, "g4_sample_top_k: softcap must be >= 0");
  if (!a.logits || !a.key || !a.token_out || !a.logp_out) return fail(G4_ERR_INVALID, "g4_sample_top_k: NULL pointer");
  if (a.split_key != 0 && a.split_key != 1) return fail(G4_ERR_INVALID, "g4_sample_top_k: split_key %d", a.split_key);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int esize = a.dtype == G4_DTYPE_BF16 ? 2 : 4;
  const bool vec = a.vocab % 8 == 0 && (a.row_stride * esize) % 16 == 0 && reinterpret_cast<uintptr_t>(a.logits) % 16 == 0;
  const dim3 grid(a.batch), block(kSampleThreads);
  if (a.dtype == G4_DTYPE_BF16) {
    if (vec)
      hipLaunchKernelGGL((sample_top_k_kernel<true, true>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((sample_top_k_kernel<true, false>), grid, block, 0, st, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((sample_top_k_kernel<false, true>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((sample_top_k_kernel<false, false>), grid, block, 0, st, a);
  }
  if (int rc = check_launch("g4_sample_top_k")) return rc;
  if (a.split_key) {
    hipLaunchKernelGGL(advance_key_kernel, dim3(1), dim3(64), 0, st, a.key);
    return check_launch("g4_sample_top_k (key split)");
  }
  return G4_OK;
}
