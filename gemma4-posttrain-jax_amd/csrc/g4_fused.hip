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
#include "g4_common.h"
#include "g4_internal.h"

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

// x * (mean(x^2) + eps)^-0.5 * w over the row held in v[] (column c = threadIdx.x + 256 * i)
template <bool BF16>
__device__ __forceinline__ void norm_row(float (&v)[kFuseMaxPerThread], int cols, const void* weight, float eps,
                                         float* red) {
  using E = Elem<BF16>;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kFuseMaxPerThread; ++i) {
    const int c = threadIdx.x + kFuseThreads * i;
    if (c < cols) ss += v[i] * v[i];
  }
  const float ms = block_sum(ss, red) / (float)cols;
  const float inv = 1.0f / sqrtf(ms + eps);
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
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cols, c = i - row * cols;
    const float g = E::load(reinterpret_cast<const T*>(gate_up), row * 2 * cols + c);
    const float u = E::load(reinterpret_cast<const T*>(gate_up), row * 2 * cols + cols + c);
    const float inner = kBeta * (g + kKappa * g * g * g);
    const float gelu = 0.5f * g * (1.0f + tanhf(inner));
    E::store(reinterpret_cast<T*>(out), i, gelu * u);
  }
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
  if (dtype == G4_DTYPE_BF16)
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
  if (dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(residual_norm_kernel<true>, dim3(rows), dim3(kFuseThreads), 0, st, cols, branch,
                       branch_weight, residual, scalar, next_weight, eps, residual_out, next_out);
  else
    hipLaunchKernelGGL(residual_norm_kernel<false>, dim3(rows), dim3(kFuseThreads), 0, st, cols, branch,
                       branch_weight, residual, scalar, next_weight, eps, residual_out, next_out);
  return check_launch("g4_residual_norm");
}

extern "C" int g4_gelu_mul(int dtype, int rows, int cols, const void* gate_up, void* out, void* stream) {
  using namespace g4;
  if (int rc = check_rows("g4_gelu_mul", dtype, rows, cols)) return rc;
  if (!gate_up || !out) return fail(G4_ERR_INVALID, "g4_gelu_mul: NULL gate_up/out");
  const int64_t n = (int64_t)rows * cols;
  if (n == 0) return G4_OK;
  const int64_t blocks64 = (n + kFuseThreads - 1) / kFuseThreads;
  const unsigned blocks = (unsigned)(blocks64 < 65536 ? blocks64 : 65536);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == G4_DTYPE_BF16)
    hipLaunchKernelGGL(gelu_mul_kernel<true>, dim3(blocks), dim3(kFuseThreads), 0, st, n, cols, gate_up, out);
  else
    hipLaunchKernelGGL(gelu_mul_kernel<false>, dim3(blocks), dim3(kFuseThreads), 0, st, n, cols, gate_up, out);
  return check_launch("g4_gelu_mul");
}
