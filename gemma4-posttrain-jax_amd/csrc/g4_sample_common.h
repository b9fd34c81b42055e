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

// Gumbel noise of element `flat` (row-major index into the [batch, K] draw) under sample_key:
// bits = xor of threefry2x32(key, (flat >> 32, flat & 0xffffffff)); u = float in [1, 2) from the
// top 23 bits minus 1, floored at the smallest normal; g = -log(-log(u)).
__device__ __forceinline__ float gumbel(uint32_t k0, uint32_t k1, uint64_t flat) {
  uint32_t x0 = (uint32_t)(flat >> 32), x1 = (uint32_t)flat;
  threefry2x32(k0, k1, x0, x1);
  const uint32_t bits = x0 ^ x1;
  const float f = __uint_as_float((bits >> 9) | 0x3F800000u) - 1.0f;
  const float u = fmaxf(kF32Tiny, f + kF32Tiny);
  return -logf(-logf(u));
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
  if (b.best > a.best || (b.best == a.best && b.idx < a.idx)) {  // ties: the first column (argmax)
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

