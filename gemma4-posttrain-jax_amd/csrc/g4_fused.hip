// Row-wise elementwise glue of the decoder layer, fused: RMSNorm, "branch norm + residual add
// (+ layer scalar) + next norm", and the gated GELU of the MLP (g4_rms_norm, g4_residual_norm,
// g4_gelu_mul).
//
// They replace chains of small framework ops (a norm alone is eight element passes) with one
// pass each, keeping the reference's rounding points: RMSNorm in f32 cast once
// (model.py:278-285), residual sums and the layer-scalar product each rounded to the activation
// dtype (model.py:505-554), gelu_tanh(gate) * up in f32 rounded once (model.py:393-396).
// One workgroup of 256 threads per row; the row is read once (kept in registers between the
// two reductions of g4_residual_norm).
#include <initializer_list>

#include "g4_common.h"
#include "g4_internal.h"

// Products and sums stay separate roundings (no multiply-add contraction), as in the reference's
// elementwise ops; the f32 paths evaluate the norm's sum of squares and x^-0.5 in f64, rounded once.
#pragma clang fp contract(off)

namespace g4 {
namespace {

constexpr int kFuseThreads = 256;
constexpr int kFuseMaxPerThread = 16;  // columns per thread held in registers: cols <= 4096

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // red may still be read by a previous reduction
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kFuseThreads / 64; ++i) s += red[i];
  return s;
}

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kFuseThreads / 64; ++i) s += red[i];
  return s;
}

// x * (mean(x^2) + eps)^-0.5 * w over the row held in v[] (column c = threadIdx.x + 256 * i).
// f32 (the parity configs): every f32 operation of the reference's formula rounded once: the
// squares, their sum (f64, then f32), / cols, + eps, x^-0.5 (f64, then f32), * r, * w.
template <bool BF16>
__device__ __forceinline__ void norm_row(float (&v)[kFuseMaxPerThread], int cols, const void* weight, float eps,
                                         float* red) {
  using E = Elem<BF16>;
  float inv;
  if constexpr (BF16) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kFuseMaxPerThread; ++i) {
      const int c = threadIdx.x + kFuseThreads * i;
      if (c < cols) ss += v[i] * v[i];
    }
    const float ms = block_sum(ss, red) / (float)cols;
    inv = 1.0f / sqrtf(ms + eps);
  } else {
    __shared__ double red64[kFuseThreads / 64];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < kFuseMaxPerThread; ++i) {
      const int c = threadIdx.x + kFuseThreads * i;
      if (c < cols) {
        const float sq = v[i] * v[i];
        ss += (double)sq;
      }
    }
    const float ms = (float)block_sum_f64(ss, red64) / (float)cols;
    inv = (float)(1.0 / sqrt((double)(ms + eps)));
  }
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    if (c < cols) {
      float y = v[i] * inv;
      if (weight) y = y * E::load(reinterpret_cast<const typename E::T*>(weight), c);
      v[i] = y;
    }
  }
}

template <bool BF16>
__global__ __launch_bounds__(kFuseThreads) void rms_norm_kernel(int cols, const void* x, const void* weight,
                                                                float eps, void* out) {
  using E = Elem<BF16>;
  using T = typename E::T;
  __shared__ float red[kFuseThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float v[kFuseMaxPerThread];
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    v[i] = c < cols ? E::load(reinterpret_cast<const T*>(x), base + c) : 0.f;
  }
  norm_row<BF16>(v, cols, weight, eps, red);
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    if (c < cols) E::store(reinterpret_cast<T*>(out), base + c, v[i]);
  }
}

// residual_out = round(round(residual + round(norm(branch) * w_branch)) * scalar)   (f32 scalar, optional)
// next_out     = round(norm(residual_out) * w_next)                                   (optional)
template <bool BF16>
__global__ __launch_bounds__(kFuseThreads) void residual_norm_kernel(int cols, const void* branch,
                                                                     const void* branch_weight,
                                                                     const void* residual, const float* scalar,
                                                                     const void* next_weight, float eps,
                                                                     void* residual_out, void* next_out) {
  using E = Elem<BF16>;
  using T = typename E::T;
  __shared__ float red[kFuseThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float v[kFuseMaxPerThread], r[kFuseMaxPerThread];
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    v[i] = c < cols ? E::load(reinterpret_cast<const T*>(branch), base + c) : 0.f;
    r[i] = c < cols ? E::load(reinterpret_cast<const T*>(residual), base + c) : 0.f;
  }
  norm_row<BF16>(v, cols, branch_weight, eps, red);
  const float s = scalar ? *scalar : 1.f;
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    float x = E::round(r[i] + E::round(v[i]));
    if (scalar) x = E::round(x * s);
    v[i] = x;
    const int c = threadIdx.x + kFuseThreads * i;
    if (c < cols) E::store(reinterpret_cast<T*>(residual_out), base + c, x);
  }
  if (!next_out) return;
  norm_row<BF16>(v, cols, next_weight, eps, red);
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    if (c < cols) E::store(reinterpret_cast<T*>(next_out), base + c, v[i]);
  }
}

// out[r, c] = round(gelu_tanh(gate[r, c]) * up[r, c]); gate_up rows are [gate (cols) | up (cols)].
template <bool BF16>
__global__ __launch_bounds__(kFuseThreads) void gelu_mul_kernel(int64_t n, int cols, const void* gate_up,
                                                                void* out) {
  using E = Elem<BF16>;
  using T = typename E::T;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cols, c = i - row * cols;
    const float g = E::load(reinterpret_cast<const T*>(gate_up), row * 2 * cols + c);
    const float u = E::load(reinterpret_cast<const T*>(gate_up), row * 2 * cols + cols + c);
    E::store(reinterpret_cast<T*>(out), i, BF16 ? gelu_tanh_mul(g, u) : gelu_tanh_mul_exact(g, u));
  }
}

// ---- bf16 rows with cols % 8 == 0: one wave per row ---------------------------------------------
// A lane owns 8-column groups lane, lane + 64, ... (16-byte loads and stores); both reductions are
// wave shuffles, so there is no LDS and no barrier. Same rounding points as the kernels above.
constexpr int kWaveGroups = 8;  // 8-column groups per lane: cols <= 64 * 8 * 8 = 4096

// The lane's groups of a weight row, loaded up front (with the data, one memory round trip).
__device__ __forceinline__ void load_weight_groups(u32x4 (&w)[kWaveGroups], int ngroups, const uint16_t* weight) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < kWaveGroups; ++j)
    if (weight && j < ngroups) w[j] = load16(weight + 8 * (lane + 64 * j));
}

// x * (mean(x^2) + eps)^-0.5 * w over the lane's groups (wave-wide mean); w from load_weight_groups
__device__ __forceinline__ void norm_groups(float (&v)[kWaveGroups][8], int ngroups, int cols,
                                            const u32x4 (&wg)[kWaveGroups], bool has_weight, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kWaveGroups; ++j)
    if (j < ngroups)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)cols + eps);
#pragma unroll
  for (int j = 0; j < kWaveGroups; ++j) {
    if (j < ngroups) {
      float w[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
      if (has_weight) unpack8(wg[j], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = has_weight ? v[j][e] * inv * w[e] : v[j][e] * inv;
    }
  }
}

__global__ __launch_bounds__(64) void rms_norm_wave_kernel(int cols, const uint16_t* x, const uint16_t* weight,
                                                           float eps, uint16_t* out) {
  const int lane = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * cols;
  const int ngroups = (cols / 8 - lane + 63) / 64;  // groups this lane owns
  float v[kWaveGroups][8];
  u32x4 wg[kWaveGroups];
  load_weight_groups(wg, ngroups, weight);
#pragma unroll
  for (int j = 0; j < kWaveGroups; ++j)
    if (j < ngroups) unpack8(load16(x + base + 8 * (lane + 64 * j)), v[j]);
  norm_groups(v, ngroups, cols, wg, weight != nullptr, eps);
#pragma unroll
  for (int j = 0; j < kWaveGroups; ++j)
    if (j < ngroups) *reinterpret_cast<u32x4*>(out + base + 8 * (lane + 64 * j)) = pack8(v[j]);
}

// ---- bf16 rows with cols % 8 == 0: 4 waves per row ----------------------------------------------
// Thread t owns the 8-column groups t, t + 256, ... (16-byte loads and stores). A reduction is a
// wave shuffle tree and one LDS exchange of the 4 wave sums; each of the two reductions has its
// own LDS slots, so one barrier each. Same rounding points as the kernels above.
constexpr int kRowThreads = 256;
constexpr int kRowGroups = 2;  // 8-column groups per thread: cols <= 256 * 8 * 2 = 4096
constexpr int kMaxNormSplits = 8;  // f32 partial rows a split-K branch may arrive in

__device__ __forceinline__ float row_sum(float v, float* red4) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
  wg_barrier();
  return (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// KS = 0: the branch is a bf16 row. KS > 0: the branch is bf16(sum of ksplit <= KS f32 partial
// rows [ksplit][rows][cols], added in split order) -- the split-K projection's output, formed here
// instead of in a separate pass.
template <int G, int KS>
__global__ __launch_bounds__(kRowThreads) void residual_norm_row_kernel(int cols, const uint16_t* branch,
                                                                        const float* partials, int ksplit,
                                                                        const uint16_t* branch_weight,
                                                                        const uint16_t* residual, const float* scalar,
                                                                        const uint16_t* next_weight, float eps,
                                                                        uint16_t* residual_out, uint16_t* next_out) {
  __shared__ float red[2][4];
  const int t = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * cols;
  const int ng = cols / 8;
  float v[G][8], r[G][8], wb[G][8], wn[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j) {  // every load of the row up front: one memory round trip
    const int g = t + kRowThreads * j;
    u32x4 a = {0u, 0u, 0u, 0u}, b = a, c = a, d = a;
    floatx4 pl[KS > 0 ? KS : 1][2];
    if (g < ng) {
      if (KS == 0) {
        a = load16(branch + base + 8 * g);
      } else {
        const int64_t plane = (int64_t)gridDim.x * cols;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          if (s < ksplit) {
            const floatx4* p = reinterpret_cast<const floatx4*>(partials + s * plane + base + 8 * g);
            pl[s][0] = p[0];
            pl[s][1] = p[1];
          }
        }
      }
      b = load16(residual + base + 8 * g);
      if (branch_weight) c = load16(branch_weight + 8 * g);
      if (next_out && next_weight) d = load16(next_weight + 8 * g);
    }
    if (KS == 0 || g >= ng) {
      unpack8(a, v[j]);
    } else {
      floatx4 lo = pl[0][0], hi = pl[0][1];
#pragma unroll
      for (int s = 1; s < KS; ++s) {
        if (s < ksplit) {
          lo += pl[s][0];
          hi += pl[s][1];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j][e] = round_bf16(lo[e]);
        v[j][4 + e] = round_bf16(hi[e]);
      }
    }
    unpack8(b, r[j]);
    unpack8(c, wb[j]);
    unpack8(d, wn[j]);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
  const float inv = 1.0f / sqrtf(row_sum(ss, red[0]) / (float)cols + eps);
  const float s = scalar ? *scalar : 1.f;
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = branch_weight ? v[j][e] * inv * wb[j][e] : v[j][e] * inv;
      float x = round_bf16(r[j][e] + round_bf16(y));
      if (scalar) x = round_bf16(x * s);
      v[j][e] = x;
    }
    const int g = t + kRowThreads * j;
    if (g < ng) *reinterpret_cast<u32x4*>(residual_out + base + 8 * g) = pack8(v[j]);
  }
  if (!next_out) return;
  ss = 0.f;
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
  const float inv2 = 1.0f / sqrtf(row_sum(ss, red[1]) / (float)cols + eps);
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = next_weight ? v[j][e] * inv2 * wn[j][e] : v[j][e] * inv2;
    const int g = t + kRowThreads * j;
    if (g < ng) *reinterpret_cast<u32x4*>(next_out + base + 8 * g) = pack8(v[j]);
  }
}

// out = round(gelu_tanh(gate) * up), 8 columns per thread per step (bf16, cols % 8 == 0)
__global__ __launch_bounds__(kFuseThreads) void gelu_mul_vec_kernel(int64_t n8, int cols8, const uint16_t* gate_up,
                                                                    uint16_t* out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cols8, c8 = i - row * cols8;
    float g[8], u[8], y[8];
    unpack8(load16(gate_up + (row * 2 * cols8 + c8) * 8), g);
    unpack8(load16(gate_up + (row * 2 * cols8 + cols8 + c8) * 8), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = gelu_tanh_mul(g[e], u[e]);
    *reinterpret_cast<u32x4*>(out + 8 * i) = pack8(y);
  }
}

// rows for the 16-byte kernels: bf16, cols a multiple of 8, 16-byte aligned arrays (NULL allowed)
bool vec_rows(int dtype, int cols, std::initializer_list<const void*> ptrs) {
  if (dtype != G4_DTYPE_BF16 || cols % 8) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return false;
  return true;
}

// ... and short enough for one wave per row
bool wave_rows(int dtype, int cols, std::initializer_list<const void*> ptrs) {
  return cols <= 64 * 8 * kWaveGroups && vec_rows(dtype, cols, ptrs);
}

int check_rows(const char* fn, int dtype, int rows, int cols) {
  if (dtype != G4_DTYPE_F32 && dtype != G4_DTYPE_BF16) return fail(G4_ERR_INVALID, "%s: dtype %d", fn, dtype);
  if (rows < 0 || cols <= 0) return fail(G4_ERR_INVALID, "%s: rows %d cols %d", fn, rows, cols);
  return G4_OK;
}

}  // namespace
}  // namespace g4

extern "C" int g4_rms_norm(int dtype, int rows, int cols, const void* x, const void* weight, float eps, void* out,
                           void* stream) {
  using namespace g4;
  if (int rc = check_rows("g4_rms_norm", dtype, rows, cols)) return rc;
  if (cols > kFuseThreads * kFuseMaxPerThread)
    return fail(G4_ERR_UNSUPPORTED, "g4_rms_norm: cols %d > %d", cols, kFuseThreads * kFuseMaxPerThread);
  if (!x || !out) return fail(G4_ERR_INVALID, "g4_rms_norm: NULL x/out");
  if (rows == 0) return G4_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (wave_rows(dtype, cols, {x, weight, out}))
    hipLaunchKernelGGL(rms_norm_wave_kernel, dim3(rows), dim3(64), 0, st, cols, reinterpret_cast<const uint16_t*>(x),
                       reinterpret_cast<const uint16_t*>(weight), eps, reinterpret_cast<uint16_t*>(out));
  else if (dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(rows), dim3(kFuseThreads), 0, st, cols, x, weight, eps, out);
  else
    hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(rows), dim3(kFuseThreads), 0, st, cols, x, weight, eps, out);
  return check_launch("g4_rms_norm");
}

extern "C" int g4_residual_norm(int dtype, int rows, int cols, const void* branch, const void* branch_weight,
                                const void* residual, const float* scalar, const void* next_weight, float eps,
                                void* residual_out, void* next_out, void* stream) {
  using namespace g4;
  if (int rc = check_rows("g4_residual_norm", dtype, rows, cols)) return rc;
  if (cols > kFuseThreads * kFuseMaxPerThread)
    return fail(G4_ERR_UNSUPPORTED, "g4_residual_norm: cols %d > %d", cols, kFuseThreads * kFuseMaxPerThread);
  if (!branch || !residual || !residual_out) return fail(G4_ERR_INVALID, "g4_residual_norm: NULL branch/residual/out");
  if (rows == 0) return G4_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (vec_rows(dtype, cols, {branch, branch_weight, residual, next_weight, residual_out, next_out}) &&
      cols <= kRowThreads * 8 * kRowGroups) {
    const auto kern = cols <= kRowThreads * 8 ? residual_norm_row_kernel<1, 0> : residual_norm_row_kernel<2, 0>;
    hipLaunchKernelGGL(kern, dim3(rows), dim3(kRowThreads), 0, st, cols, reinterpret_cast<const uint16_t*>(branch),
                       (const float*)nullptr, 0, reinterpret_cast<const uint16_t*>(branch_weight),
                       reinterpret_cast<const uint16_t*>(residual),
                       scalar, reinterpret_cast<const uint16_t*>(next_weight), eps,
                       reinterpret_cast<uint16_t*>(residual_out), reinterpret_cast<uint16_t*>(next_out));
  } else if (dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(residual_norm_kernel<true>, dim3(rows), dim3(kFuseThreads), 0, st, cols, branch,
                       branch_weight, residual, scalar, next_weight, eps, residual_out, next_out);
  else
    hipLaunchKernelGGL(residual_norm_kernel<false>, dim3(rows), dim3(kFuseThreads), 0, st, cols, branch,
                       branch_weight, residual, scalar, next_weight, eps, residual_out, next_out);
  return check_launch("g4_residual_norm");
}

extern "C" int g4_residual_norm_splitk(int rows, int cols, const float* partials, int ksplit,
                                       const void* branch_weight, const void* residual, const float* scalar,
                                       const void* next_weight, float eps, void* residual_out, void* next_out,
                                       void* stream) {
  using namespace g4;
  if (int rc = check_rows("g4_residual_norm_splitk", G4_DTYPE_BF16, rows, cols)) return rc;
  if (ksplit < 1 || ksplit > kMaxNormSplits)
    return fail(G4_ERR_UNSUPPORTED, "g4_residual_norm_splitk: ksplit %d (1..%d)", ksplit, kMaxNormSplits);
  if (!partials || !residual || !residual_out)
    return fail(G4_ERR_INVALID, "g4_residual_norm_splitk: NULL partials/residual/out");
  if (!vec_rows(G4_DTYPE_BF16, cols, {branch_weight, residual, next_weight, residual_out, next_out}) ||
      (reinterpret_cast<uintptr_t>(partials) & 15) || cols > kRowThreads * 8 * kRowGroups)
    return fail(G4_ERR_UNSUPPORTED,
                "g4_residual_norm_splitk: cols %d (a multiple of 8, <= %d) and 16-byte aligned rows needed", cols,
                kRowThreads * 8 * kRowGroups);
  if (rows == 0) return G4_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto kern = cols <= kRowThreads * 8 ? residual_norm_row_kernel<1, kMaxNormSplits>
                                            : residual_norm_row_kernel<2, kMaxNormSplits>;
  hipLaunchKernelGGL(kern, dim3(rows), dim3(kRowThreads), 0, st, cols, (const uint16_t*)nullptr, partials, ksplit,
                     reinterpret_cast<const uint16_t*>(branch_weight), reinterpret_cast<const uint16_t*>(residual),
                     scalar, reinterpret_cast<const uint16_t*>(next_weight), eps,
                     reinterpret_cast<uint16_t*>(residual_out), reinterpret_cast<uint16_t*>(next_out));
  return check_launch("g4_residual_norm_splitk");
}

extern "C" int g4_gelu_mul(int dtype, int rows, int cols, const void* gate_up, void* out, void* stream) {
  using namespace g4;
  if (int rc = check_rows("g4_gelu_mul", dtype, rows, cols)) return rc;
  if (!gate_up || !out) return fail(G4_ERR_INVALID, "g4_gelu_mul: NULL gate_up/out");
  const int64_t n = (int64_t)rows * cols;
  if (n == 0) return G4_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (vec_rows(dtype, cols, {gate_up, out})) {
    const int64_t n8 = n / 8;
    const int64_t b8 = (n8 + kFuseThreads - 1) / kFuseThreads;
    hipLaunchKernelGGL(gelu_mul_vec_kernel, dim3((unsigned)(b8 < 65536 ? b8 : 65536)), dim3(kFuseThreads), 0, st, n8,
                       cols / 8, reinterpret_cast<const uint16_t*>(gate_up), reinterpret_cast<uint16_t*>(out));
    return check_launch("g4_gelu_mul");
  }
  const int64_t blocks64 = (n + kFuseThreads - 1) / kFuseThreads;
  const unsigned blocks = (unsigned)(blocks64 < 65536 ? blocks64 : 65536);
  if (dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(gelu_mul_kernel<true>, dim3(blocks), dim3(kFuseThreads), 0, st, n, cols, gate_up, out);
  else
    hipLaunchKernelGGL(gelu_mul_kernel<false>, dim3(blocks), dim3(kFuseThreads), 0, st, n, cols, gate_up, out);
  return check_launch("g4_gelu_mul");
}
