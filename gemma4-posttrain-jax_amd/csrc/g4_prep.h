// Per-vector preparation shared by g4_kv_append and the decode kernels that fuse it: one wave
// prepares one head vector of D elements (q, k or v of one token), lane l owning elements
// [l*D/64, (l+1)*D/64) (D >= 64; lane l < D owns d = l below that), so a RoPE partner (d +- D/2)
// is lane l ^ 32 in the same register. Replaces forward_rms_norm (model.py:278-285) and
// forward_rotary_embedding (model.py:309-317) on one row of forward_attention (model.py:463-482).
#pragma once

#include "g4_common.h"

namespace g4 {

// PER consecutive elements in one access (PER = 2, 4 or 8; the address aligned to the access)
template <int PER>
__device__ __forceinline__ void ld_bf16(const uint16_t* p, float (&x)[PER]) {
  uint32_t w[PER / 2];
  if constexpr (PER == 2) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (PER == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x, w[1] = v.y;
  } else {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = v[i];
  }
#pragma unroll
  for (int i = 0; i < PER / 2; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <int PER>
__device__ __forceinline__ void st_bf16(uint16_t* p, const float (&x)[PER]) {
  uint32_t w[PER / 2];
#pragma unroll
  for (int i = 0; i < PER / 2; ++i) w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
  if constexpr (PER == 2) {
    *reinterpret_cast<uint32_t*>(p) = w[0];
  } else if constexpr (PER == 4) {
    *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  } else {
    *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

template <int PER>
__device__ __forceinline__ void ld_f32(const float* p, float (&x)[PER]) {
#pragma unroll
  for (int i = 0; i < PER; i += 2) {
    if constexpr (PER == 2) {
      const float2 v = *reinterpret_cast<const float2*>(p);
      x[0] = v.x, x[1] = v.y;
    } else if (i % 4 == 0) {
      const float4 v = *reinterpret_cast<const float4*>(p + i);
      x[i] = v.x, x[i + 1] = v.y, x[i + 2] = v.z, x[i + 3] = v.w;
    }
  }
}


// The loads of one vector (its elements, norm weights and cos / sin row), all issued before any
// arithmetic: one memory round trip. VEC: bf16, D >= 128, rows aligned to one lane's D/64 elements
// (checked on the host).
template <bool BF16, int D>
struct PrepIn {
  static constexpr int PER = D >= 64 ? D / 64 : 1;
  float x[PER], wv[PER], cv[PER], sv[PER];
};

template <bool BF16, int D, bool VEC>
__device__ __forceinline__ void prep_load(PrepIn<BF16, D>& in, const typename Elem<BF16>::T* src,
                                          const typename Elem<BF16>::T* w, bool rope, const float* rcos,
                                          const float* rsin, int lane) {
  using E = Elem<BF16>;
  constexpr int PER = PrepIn<BF16, D>::PER;
  const bool lane_on = D >= 64 || lane < D;
  if constexpr (VEC) {
    ld_bf16<PER>(reinterpret_cast<const uint16_t*>(src) + lane * PER, in.x);
#pragma unroll
    for (int e = 0; e < PER; ++e) in.wv[e] = 1.f, in.cv[e] = in.sv[e] = 0.f;
    if (w) ld_bf16<PER>(reinterpret_cast<const uint16_t*>(w) + lane * PER, in.wv);
    if (rope) {
      ld_f32<PER>(rcos + lane * PER, in.cv);
      ld_f32<PER>(rsin + lane * PER, in.sv);
    }
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int d = lane * PER + e;
      in.x[e] = lane_on ? E::load(src, d) : 0.f;
      in.wv[e] = (w && lane_on) ? E::load(w, d) : 1.f;
      in.cv[e] = (rope && lane_on) ? rcos[d] : 0.f;
      in.sv[e] = (rope && lane_on) ? rsin[d] : 0.f;
    }
  }
}

// RMSNorm and RoPE of the loaded vector with the reference's rounding points; the result in in.x.
template <bool BF16, int D>
__device__ __forceinline__ void prep_math(PrepIn<BF16, D>& in, bool norm, bool has_w, bool rope, float eps) {
  using E = Elem<BF16>;
  constexpr int PER = PrepIn<BF16, D>::PER;
  constexpr int PARTNER = D >= 64 ? 32 : D / 2;
  const int lane = threadIdx.x & 63;
  if (norm) {
    // forward_rms_norm (model.py:278-285): f32 statistics, x * (mean(x^2) + eps)^-0.5 * w. f32
    // vectors (the parity configs): each f32 operation rounded once, the sum of the squares and
    // x^-0.5 evaluated in f64.
#pragma clang fp contract(off)
    float inv;
    if constexpr (BF16) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < PER; ++e) ss += in.x[e] * in.x[e];
      ss = wave_sum(ss);
      inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
    } else {
      double ss = 0.0;
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const float sq = in.x[e] * in.x[e];
        ss += (double)sq;
      }
      for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
      inv = (float)(1.0 / sqrt((double)((float)ss / (float)D + eps)));
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      float y = in.x[e] * inv;
      if (has_w) y = y * in.wv[e];
      in.x[e] = E::round(y);
    }
  }

  if (rope) {
    // x*cos + rotate_half(x)*sin with cos/sin first rounded to the activation dtype
    // (model.py:309-317); products and sum are rounded separately (no FMA contraction).
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int d = lane * PER + e;
      const float partner = __shfl_xor(in.x[e], PARTNER, 64);
      const float rot = d < D / 2 ? -partner : partner;
      const float c = E::round(in.cv[e]);
      const float sn = E::round(in.sv[e]);
      const float t0 = in.x[e] * c;  // plain operators: the pragma above keeps them unfused
      const float t1 = rot * sn;
      in.x[e] = E::round(t0 + t1);
    }
  }
}

// prep_load + prep_math; x receives the prepared vector.
template <bool BF16, int D, bool VEC>
__device__ __forceinline__ void prep_head(const typename Elem<BF16>::T* src, const typename Elem<BF16>::T* w,
                                          bool norm, bool rope, const float* rcos, const float* rsin, float eps,
                                          int lane, float (&x)[D >= 64 ? D / 64 : 1]) {
  PrepIn<BF16, D> in;
  prep_load<BF16, D, VEC>(in, src, w, rope, rcos, rsin, lane);
  prep_math<BF16, D>(in, norm, w != nullptr, rope, eps);
#pragma unroll
  for (int e = 0; e < PrepIn<BF16, D>::PER; ++e) x[e] = in.x[e];
}

}  // namespace g4
