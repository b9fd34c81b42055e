// Sampling helpers shared by g4_sample.hip (the sampler over materialized logits) and
// g4_lm_head.hip (the LM head with the sampler in its epilogue); included inside namespace g4::{anon}.
//
// The random stream is JAX's: threefry2x32 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011; 20 rounds, the Skein rotation constants), key splitting and random bits
// in JAX's partitionable layout, uniform floats from the top 23 bits, Gumbel noise -log(-log(u)) and
// categorical = argmax(scores + noise).
#pragma once

constexpr float kF32Tiny = 1.17549435e-38f;  // smallest normal float: uniform's minval

__device__ __forceinline__ uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// threefry2x32 with 20 rounds: key schedule (k0, k1, k0 ^ k1 ^ 0x1BD11BDA) injected after every
// four rounds together with the injection count; rotations 13 15 26 6 / 17 29 16 24.
__device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1, uint32_t& x0, uint32_t& x1) {
  const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  constexpr int rot[2][4] = {{13, 15, 26, 6}, {17, 29, 16, 24}};
  x0 += ks[0];
  x1 += ks[1];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x0 += x1;
      x1 = rotl32(x1, rot[i & 1][j]) ^ x0;
    }
    x0 += ks[(i + 1) % 3];
    x1 += ks[(i + 2) % 3] + (uint32_t)(i + 1);
  }
}

// Natural log of a positive, normal, finite x: log2(x) from v_log_f32, times ln 2 held as
// kLn2Hi + kLn2Lo, with the rounding error of y * kLn2Hi recovered by an fma (Dekker's product).
// On that domain this is the device library's logf, which adds only the scaling of subnormal
// arguments and the selects for 0, inf and NaN; both logs of the Gumbel noise stay in it
// (u >= 2^-126, and -log(u) >= -log(1 - 2^-23) > 2^-24).
constexpr float kLn2Hi = 0x1.62e42ep-1f;  // ln 2 rounded to 24 bits
constexpr float kLn2Lo = 0x1.efa39ep-25f;  // ln 2 - kLn2Hi

__device__ __forceinline__ float log_pos_normal(float x) {
  const float y = __builtin_amdgcn_logf(x);
  const float hi = y * kLn2Hi;
  return fmaf(kLn2Hi, y, fmaf(kLn2Lo, y, fmaf(y, kLn2Hi, -hi)));
}

// Gumbel noise of element `flat` (row-major index into the [batch, K] draw) under sample_key:
// bits = xor of threefry2x32(key, (flat >> 32, flat & 0xffffffff)); u = float in [1, 2) from the
// top 23 bits minus 1, floored at the smallest normal; g = -log(-log(u)).
__device__ __forceinline__ float gumbel(uint32_t k0, uint32_t k1, uint64_t flat) {
  uint32_t x0 = (uint32_t)(flat >> 32), x1 = (uint32_t)flat;
  threefry2x32(k0, k1, x0, x1);
  const uint32_t bits = x0 ^ x1;
  const float f = __uint_as_float((bits >> 9) | 0x3F800000u) - 1.0f;
  const float u = fmaxf(kF32Tiny, f + kF32Tiny);
  return -log_pos_normal(-log_pos_normal(u));
}

// The running argmax under jnp.argmax's rule (argmax in _sample_token and inside
// jax.random.categorical): a NaN score is greater than every number and the first NaN column wins.
// takes_best: a score met after every column of `best` replaces it (columns arrive in increasing
// order, so an equal score keeps the earlier column, and a NaN best is never replaced).
__device__ __forceinline__ bool takes_best(float score, float best) { return !(score <= best) && best == best; }

// beats: whether state (bb, bi) wins over (ab, ai) when two states of disjoint columns merge.
__device__ __forceinline__ bool beats(float bb, int bi, float ab, int ai) {
  const bool bn = bb != bb, an = ab != ab;
  if (bn || an) return bn && (!an || bi < ai);
  return bb > ab || (bb == ab && bi < ai);
}

struct RowState {
  float m, s;  // running max of x and sum of exp(x - m)
  float best;  // best score so far
  int idx;     // its column
};

__device__ __forceinline__ void merge(RowState& a, const RowState& b) {
  if (b.m > a.m) {
    a.s = a.s * expf(a.m - b.m) + b.s;
    a.m = b.m;
  } else if (b.m > kF32Min) {
    a.s += b.s * expf(b.m - a.m);
  }
  if (beats(b.best, b.idx, a.best, a.idx)) {  // ties and NaNs: the first column (argmax)
    a.best = b.best;
    a.idx = b.idx;
  }
}

__device__ __forceinline__ RowState shfl_state(const RowState& x, int mask) {
  RowState y;
  y.m = __shfl_xor(x.m, mask, 64);
  y.s = __shfl_xor(x.s, mask, 64);
  y.best = __shfl_xor(x.best, mask, 64);
  y.idx = __shfl_xor(x.idx, mask, 64);
  return y;
}


// The soft-cap of a bf16 value x, bf16(tanh(x / cap) * cap) with the division, tanhf and the
// multiply in f32, through a table of the 16 binades where it is neither x nor saturated. With
// e_c = floor(log2(cap)):
// - 2^(e_c - 125) <= |x| < 2^(e_c - 12): y = x / cap is a normal float below 2^-12, so
//   tanh(y) = y (1 - y^2 / 3 + ...) moves x by less than 2^-21 relative after the f32 roundings, far
//   below half a bf16 ulp (2^-9): the result is x (smaller x would make y subnormal or zero);
// - 2^(e_c - 12) <= |x| < 2^(e_c + 4): the table, 2 signs x 16 binades x 128 mantissas, filled with
//   the formula itself;
// - |x| >= 2^(e_c + 4) (y > 8), inf, NaN and |x| < 2^(e_c - 125): the formula itself (rare: a
//   lane-divergent branch).
constexpr int kCapTableEntries = 4096;

typedef __attribute__((address_space(3))) const uint16_t LdsU16;

struct CapTable {
  const LdsU16* tab;  // LDS: entry (sign << 11) | (binade << 7) | mantissa
  int e0;             // biased exponent of binade 0 (>= 1)
  int e_id;           // smallest biased exponent of the identity range
  float cap;
};

__device__ __forceinline__ float softcap_formula(float x, float cap) {
  return round_bf16(tanhf(x / cap) * cap);  // the reference divides by the cap
}

__device__ __forceinline__ CapTable cap_table(const void* lds_tab, float cap) {
  const int ec = (int)((__float_as_uint(cap) >> 23) & 0xff);
  CapTable t;
  t.tab = (const LdsU16*)lds_tab;
  t.e0 = ec - 12 < 1 ? 1 : ec - 12;
  t.e_id = ec - 125 < 1 ? 1 : ec - 125;
  t.cap = cap;
  return t;
}

// Fills the table with threads tid, tid + nthreads, ... (the caller synchronizes before use).
__device__ __forceinline__ void cap_table_fill(uint16_t* tab, float cap, int tid, int nthreads) {
  const int e0 = cap_table(tab, cap).e0;
  for (int i = tid; i < kCapTableEntries; i += nthreads) {
    const int e = e0 + ((i >> 7) & 15);
    const uint32_t bits = ((uint32_t)(i >> 11) << 15) | ((uint32_t)(e < 255 ? e : 255) << 7) | (uint32_t)(i & 127);
    tab[i] = (uint16_t)f32_to_bf16_bits(softcap_formula(bf16_bits_to_f32(bits), cap));
  }
}

__device__ __forceinline__ float capped(uint32_t bits, const CapTable& t) {
  const uint32_t mag = bits & 0x7fffu;
  const int e = (int)(mag >> 7), rel = e - t.e0;
  if (rel < 0 && e >= t.e_id) return bf16_bits_to_f32(bits);
  if (rel >= 0 && rel < 16) return bf16_bits_to_f32(t.tab[((bits >> 15) << 11) | ((uint32_t)rel << 7) | (mag & 127u)]);
  return softcap_formula(bf16_bits_to_f32(bits), t.cap);
}
