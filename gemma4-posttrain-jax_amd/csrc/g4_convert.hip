// Rollout weight handoff: the f32 master -> bf16 rollout cast and its exact inverse
// (g4_convert_f32_to_bf16, g4_convert_bf16_to_f32).
//
// The narrowing is the reference's integer round-to-nearest-even (inference_device.py:21-25):
// bf16 = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 on the raw f32 bits, which keeps signed zeros
// and bf16 subnormals (no flush to zero) and matches XLA's f32 -> bf16 convert on finite values
// (sharding.py:200-228 casts with astype). The finiteness check follows the same lines: an input
// whose exponent is all ones (inf / NaN) or a result that rounded up to the all-ones exponent
// (overflow) sets the caller's flag. HBM-bound: 8 elements per thread per step, 32-byte loads.
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kConvThreads = 256;

__device__ __forceinline__ uint32_t rne_bf16(uint32_t bits) { return (bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16; }

__device__ __forceinline__ bool nonfinite_pair(uint32_t bits, uint32_t r) {
  return (bits & 0x7F800000u) == 0x7F800000u || (r & 0x7F80u) == 0x7F80u;
}

__global__ __launch_bounds__(kConvThreads) void f32_to_bf16_kernel(const uint32_t* in, uint16_t* out, int64_t n,
                                                                   int32_t* nonfinite) {
  bool bad = false;
  const int64_t n8 = n / 8;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += step) {
    const uint4 a = reinterpret_cast<const uint4*>(in)[2 * i];
    const uint4 b = reinterpret_cast<const uint4*>(in)[2 * i + 1];
    const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r[e] = rne_bf16(v[e]);
      bad = bad || nonfinite_pair(v[e], r[e]);
    }
    reinterpret_cast<uint4*>(out)[i] = make_uint4(r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16),
                                                  r[6] | (r[7] << 16));
  }
  for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {  // the tail
    const uint32_t r = rne_bf16(in[i]);
    bad = bad || nonfinite_pair(in[i], r);
    out[i] = (uint16_t)r;
  }
  if (bad && nonfinite) *nonfinite = 1;  // same value from every writer: no atomic needed
}

__global__ __launch_bounds__(kConvThreads) void bf16_to_f32_kernel(const uint16_t* in, uint32_t* out, int64_t n) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) out[i] = (uint32_t)in[i] << 16;
}

unsigned conv_blocks(int64_t work) {
  const int64_t b = (work + kConvThreads - 1) / kConvThreads;
  return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

}  // namespace
}  // namespace g4

extern "C" int g4_convert_f32_to_bf16(const float* in, void* out, int64_t n, int32_t* nonfinite, void* stream) {
  using namespace g4;
  if (n < 0) return fail(G4_ERR_INVALID, "g4_convert_f32_to_bf16: n %lld", (long long)n);
  if (n == 0) return G4_OK;
  if (!in || !out) return fail(G4_ERR_INVALID, "g4_convert_f32_to_bf16: NULL in/out");
  if ((reinterpret_cast<uintptr_t>(in) & 15) || (reinterpret_cast<uintptr_t>(out) & 15))
    return fail(G4_ERR_INVALID, "g4_convert_f32_to_bf16: in and out must be 16-byte aligned");
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(conv_blocks(n / 8 > 0 ? n / 8 : n)), dim3(kConvThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(in),
                     reinterpret_cast<uint16_t*>(out), n, nonfinite);
  return check_launch("g4_convert_f32_to_bf16");
}

extern "C" int g4_convert_bf16_to_f32(const void* in, float* out, int64_t n, void* stream) {
  using namespace g4;
  if (n < 0) return fail(G4_ERR_INVALID, "g4_convert_bf16_to_f32: n %lld", (long long)n);
  if (n == 0) return G4_OK;
  if (!in || !out) return fail(G4_ERR_INVALID, "g4_convert_bf16_to_f32: NULL in/out");
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(conv_blocks(n)), dim3(kConvThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint16_t*>(in),
                     reinterpret_cast<uint32_t*>(out), n);
  return check_launch("g4_convert_bf16_to_f32");
}
