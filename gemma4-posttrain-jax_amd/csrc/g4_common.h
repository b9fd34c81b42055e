// Device helpers shared by the gfx950 kernels: bf16 rounding, element access, MFMA types,
// wavefront reductions, and the ring-slot arithmetic of model.py:355-357.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace g4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// jnp.finfo(bf16).min / jnp.finfo(f32).min: the masked-score fill value (model.py:497).
constexpr float kBf16Min = -3.3895313892515355e38f;
constexpr float kF32Min = -3.4028234663852886e38f;

// Value-cache layout: per (b, kv head) a [slot_stride / 8][D][8] block. The 8 consecutive slots of
// one value dim are contiguous (16 bytes in bf16: one MFMA operand, read with one 16-byte load), and
// one slot's D values lie inside one 8*D-element span (4 KiB for bf16, D = 256), so appending a slot
// touches D / 8 cache lines of 128 bytes rather than D.
__host__ __device__ __forceinline__ int64_t vt_index(int64_t slot, int d, int D) {
  return ((slot >> 3) * D + d) * 8 + (slot & 7);
}

// Key-cache layout: per (b, kv head) a [slot_stride / 32][D / KR][2][16][KR] block, KR = min(D, 32)
// dims per run. A 32-slot chunk's keys sit in the order of the decode / prefill MFMA's A operand:
// block (chunk, s, bb) holds, for each of the 16 lanes col = 4 (r >> 3) + (r & 3), key slot
// 32 chunk + r, r = 8 (col >> 2) + 4 bb + (col & 3), dims [KR s, KR s + KR). One MFMA operand load
// (16 lanes x 4 groups of 8 dims, D >= 32) then reads one contiguous KiB (bf16), and one slot's D
// values are D / KR runs of KR elements.
__host__ __device__ __forceinline__ int64_t kt_index(int64_t slot, int d, int D) {
  const int kr = D < 32 ? D : 32;
  const int r = (int)(slot & 31);
  const int col = ((r >> 3) << 2) | (r & 3);
  return ((((slot >> 5) * (D / kr) + d / kr) * 2 + ((r >> 2) & 1)) * 16 + col) * kr + d % kr;
}

// Byte offset (bf16) of the 16-byte operand of value dim d, slots [8 g, 8 g + 8).
__host__ __device__ __forceinline__ uint32_t vt_operand_bytes(int g, int d, int D) {
  return ((uint32_t)g * (uint32_t)D + (uint32_t)d) * 16u;
}

__host__ __device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(b << 16);
#else
  union { uint32_t u; float f; } c;
  c.u = b << 16;
  return c.f;
#endif
}

// float32 -> bf16 bits, round to nearest even: gfx950's conversion instruction (v_cvt_pk_bf16_f32),
// the same bits as the integer formula (u + 0x7fff + ((u >> 16) & 1)) >> 16 for every non-NaN
// input, subnormals included; NaN stays a quiet NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// two floats -> one packed bf16 pair (lo in bits 0..15), one conversion instruction
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Element access for the two storage types (bf16 as raw uint16 bits, f32 as float).
template <bool BF16> struct Elem;
template <> struct Elem<true> {
  typedef uint16_t T;
  static constexpr float kMin = kBf16Min;
  __device__ static __forceinline__ float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ static __forceinline__ void store(T* p, int64_t i, float v) { p[i] = (uint16_t)f32_to_bf16_bits(v); }
  __device__ static __forceinline__ float round(float v) { return round_bf16(v); }
};
template <> struct Elem<false> {
  typedef float T;
  static constexpr float kMin = kF32Min;
  __device__ static __forceinline__ float load(const T* p, int64_t i) { return p[i]; }
  __device__ static __forceinline__ void store(T* p, int64_t i, float v) { p[i] = v; }
  __device__ static __forceinline__ float round(float v) { return v; }
};

// Wave64 reductions over lanes that differ in the given xor masks.
__device__ __forceinline__ float wave_sum(float v) {
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Ring slot r of a Wc-slot buffer holds the greatest position p <= last with p % Wc == r
// (model.py:357); negative means never written.
__host__ __device__ __forceinline__ int64_t ring_slot_position(int64_t last, int64_t slot, int64_t wc) {
  int64_t diff = last - slot;
  int64_t q = diff >= 0 ? diff / wc : -((-diff + wc - 1) / wc);  // floor division
  return slot + q * wc;
}

__host__ __device__ __forceinline__ int64_t floor_mod(int64_t a, int64_t m) {
  int64_t r = a % m;
  return r < 0 ? r + m : r;
}

// Workgroup barrier after this wave's LDS writes complete, without waiting for vector memory:
// __syncthreads()'s release fence would also wait for in-flight LDS DMA (buffer_load ... lds).
__device__ __forceinline__ void wg_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte global load / store of 8 bf16 values (raw bits).
__device__ __forceinline__ u32x4 load16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// gelu_tanh(g) * u in f32 (model.py:393-396; jax.nn.gelu(approximate=True)), g and u already
// rounded to the activation dtype; shared by the MLP activation kernel and the gate/up epilogue.
__device__ __forceinline__ float gelu_tanh_mul(float g, float u) {
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  const float inner = kBeta * (g + kKappa * g * g * g);
  return 0.5f * g * (1.0f + tanhf(inner)) * u;
}

// exp(x) of an f32 value evaluated in f64 and rounded once to f32 (the f32 kernels' softmax).
__device__ __forceinline__ float exp_f32_exact(float x) { return (float)exp((double)x); }

// gelu_tanh(g) * u of an f32 model, each f32 operation of jax.nn.gelu(approximate=True) rounded
// once in its own order, x * (0.5 * (1 + tanh(c * (x + 0.044715 * ((x * x) * x))))), with tanh
// evaluated in f64 (the exactly rounded evaluation the fp32 parity configs are checked against).
__device__ __forceinline__ float gelu_tanh_mul_exact(float g, float u) {
#pragma clang fp contract(off)
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi) rounded to f32
  const float x3 = (g * g) * g;
  const float inner = kBeta * (g + 0.044715f * x3);
  const float th = (float)tanh((double)inner);
  const float gel = g * (0.5f * (1.0f + th));
  return gel * u;
}

// 16-byte LDS read issued from inline assembly, for operand tiles that buffer_load ... lds fills:
// the compiler does not see the read, so it adds no wait for DMAs in flight into other buffers (it
// cannot always tell them apart and then waits for all of them). The caller orders the read after
// its own wait for the tile's DMA and waits for the read with lgkm_wait before using the value.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
  u32x4 v;
  __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// s_waitcnt lgkmcnt(n), tied to `v` so that no use of v is scheduled before it (n a constant once
// the caller's loop is unrolled; LDS reads complete in issue order).
__device__ __forceinline__ void lgkm_wait(int n, u32x4& v) {
  switch (n) {
    case 0: __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(v)); break;
    case 1: __asm__ volatile("s_waitcnt lgkmcnt(1)" : "+v"(v)); break;
    case 2: __asm__ volatile("s_waitcnt lgkmcnt(2)" : "+v"(v)); break;
    case 3: __asm__ volatile("s_waitcnt lgkmcnt(3)" : "+v"(v)); break;
    case 4: __asm__ volatile("s_waitcnt lgkmcnt(4)" : "+v"(v)); break;
    case 5: __asm__ volatile("s_waitcnt lgkmcnt(5)" : "+v"(v)); break;
    case 6: __asm__ volatile("s_waitcnt lgkmcnt(6)" : "+v"(v)); break;
    default: __asm__ volatile("s_waitcnt lgkmcnt(7)" : "+v"(v)); break;
  }
}

// 8 bf16 values (one 16-byte word) <-> 8 floats (exact widening; narrowing rounds to nearest even).
__device__ __forceinline__ void unpack8(u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = __uint_as_float(w[q] << 16);
    f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
}

// Raw buffer access (gfx9 resource word 3 = 0x00020000): base and size live in SGPRs, each lane
// supplies a 32-bit byte offset, and a uniform offset rides in soffset. Reads at or beyond
// `bytes` return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, (int)soffset, 0));
}

// Cache-policy bits of a non-temporal access (the nt bit), for streams of which each byte is read
// by one workgroup once: the value cache, and the key cache where no other workgroup reads the same
// rows. On the decode streams nt loads measured 5-7 % faster than plain ones (config 2: 16.3 -> 15.4
// us with nt on V only; the E2B two-launch layer: 60.6 -> 56.4 us with nt on K and V). Where the two
// workgroups of a pair read the same K rows (the second from L2), plain loads stay faster.
constexpr int kNonTemporal = 2;

__device__ __forceinline__ u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, (int)soffset, kNonTemporal));
}

__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace g4
