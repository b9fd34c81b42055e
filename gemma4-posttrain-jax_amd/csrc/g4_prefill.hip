// Causal / sliding-window prefill attention on the prompt chunk's own K/V (g4_prefill_attention).
//
// Replaces make_qk_masks + the attention einsums of gemma4_posttrain_jax/model.py:320-335,
// 496-499 in prefill mode (model.py:455-457, 621-623). Query rows of one kv head are the
// (position, r) pairs; a wave owns 16 rows = 16/R consecutive positions x R heads, so all its
// rows share one key range. Scores come from MFMA 16x16x32 with key rows as the A operand and
// the 16 query rows as B (the transposed product S^T), which leaves each lane holding one row's
// scores for 8 consecutive keys — the B-operand layout of the O^T = V^T P^T product, fed by
// 16-byte loads along keys from the transposed value buffer.
// The reference rounds probabilities after an f32 softmax over the full row; to reproduce that
// rounding the kernel makes two passes over the key range: pass 1 finds each row's max and
// sum, pass 2 recomputes the scores and forms exact bf16 probabilities for the value product.
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kPrefillWaves = 4;

__device__ __forceinline__ bool prefill_valid(const G4PrefillArgs& a, const uint8_t* km, int row_pos, int key) {
  if (key >= a.seq || key > row_pos) return false;
  if (a.window > 0 && key <= row_pos - a.window) return false;
  return km[key] != 0;
}

template <int D>
__global__ __launch_bounds__(kPrefillWaves * 64) void prefill_bf16_kernel(G4PrefillArgs a) {
  constexpr int KS = D / 32;
  constexpr int DB = D / 16;
  const int R = a.group;
  const int ppw = 16 / R;  // positions per wave
  const int S = a.seq, H = a.kv_heads;
  const int b = blockIdx.z, h = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int pos0 = (blockIdx.x * kPrefillWaves + w) * ppw;
  if (pos0 >= S) return;  // no barriers in this kernel: idle waves may leave early

  const int my_pos = pos0 + col / R;
  const int r = col - (col / R) * R;
  const bool row_ok = my_pos < S;
  const int64_t bh = (int64_t)b * H + h;
  const uint8_t* km = a.key_mask + (int64_t)b * a.key_mask_stride;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) + bh * a.k_stride * D;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.vt) + bh * D * a.k_stride;

  bf16x8 qop[KS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + ((((int64_t)b * S + my_pos) * H + h) * R + r) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row_ok) v = load16(qrow + 32 * s + 8 * grp);
      qop[s] = as_bf16x8(v);
    }
  }

  const int pos_max = min(pos0 + ppw - 1, S - 1);
  const int kmin = a.window > 0 ? max(0, pos0 - a.window + 1) : 0;
  const int c_begin = kmin >> 5, c_end = pos_max >> 5;

  auto scores = [&](int c0, floatx4 (&acc)[2]) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const uint16_t* kp = kbase + kt_index(c0 + 8 * (col >> 2) + 4 * bb + (col & 3), 8 * grp, D);
      u32x4 kv[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) kv[s] = load16(kp + 1024 * s);  // dims 32 s + 8 grp .. + 7
      floatx4 acc_b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc_b = mfma16x16x32(as_bf16x8(kv[s]), qop[s], acc_b);
      acc[bb] = acc_b;
    }
  };

  // ---- pass 1: row max and sum ------------------------------------------------------------------
  float m = kBf16Min, l = 0.f;
  for (int c = c_begin; c <= c_end; ++c) {
    const int c0 = c << 5;
    floatx4 acc[2];
    scores(c0, acc);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = c0 + 8 * grp + 4 * bb + j;
        const float s = (row_ok && prefill_valid(a, km, my_pos, key)) ? round_bf16(acc[bb][j]) : kBf16Min;
        if (s > m) {
          l = l * expf(m - s) + 1.f;
          m = s;
        } else {
          l += expf(s - m);
        }
      }
    }
  }
#pragma unroll
  for (int msk = 16; msk <= 32; msk <<= 1) {
    const float m2 = __shfl_xor(m, msk, 64);
    const float l2 = __shfl_xor(l, msk, 64);
    const float mm = fmaxf(m, m2);
    l = l * expf(m - mm) + l2 * expf(m2 - mm);
    m = mm;
  }
  // A row with no valid key is the reference's softmax over S equal fills: 1/S on every key.
  const bool row_masked = row_ok && m == kBf16Min;
  const bool any_masked = __any(row_masked);
  const float p_uniform = round_bf16(1.0f / (float)S);
  const int c2_begin = any_masked ? 0 : c_begin;
  const int c2_end = any_masked ? (S - 1) >> 5 : c_end;

  // ---- pass 2: exact probabilities and O^T = V^T P^T ---------------------------------------------
  floatx4 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c = c2_begin; c <= c2_end; ++c) {
    const int c0 = c << 5;
    const int kb = c0 + 8 * grp;
    u32x4 vv[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) vv[i] = load16(vbase + vt_index(kb, 16 * i + col, D));
    floatx4 acc[2];
    scores(c0, acc);
    uint32_t pw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * bb + j;
        const int key = kb + e;
        float p = 0.f;
        if (row_masked) {
          p = key < S ? p_uniform : 0.f;
        } else if (row_ok && prefill_valid(a, km, my_pos, key)) {
          p = round_bf16(expf(round_bf16(acc[bb][j]) - m) / l);
        }
        pw[e >> 1] |= f32_to_bf16_bits(p) << (16 * (e & 1));
      }
    }
    const bf16x8 pop = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
#pragma unroll
    for (int i = 0; i < DB; ++i) oacc[i] = mfma16x16x32(as_bf16x8(vv[i]), pop, oacc[i]);
  }

  if (row_ok) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((((int64_t)b * S + my_pos) * H + h) * R + r) * D;
#pragma unroll
    for (int i = 0; i < DB; ++i) {
      const uint32_t w0 = f32_to_bf16_bits(oacc[i][0]) | (f32_to_bf16_bits(oacc[i][1]) << 16);
      const uint32_t w1 = f32_to_bf16_bits(oacc[i][2]) | (f32_to_bf16_bits(oacc[i][3]) << 16);
      *reinterpret_cast<uint2*>(orow + 16 * i + 4 * grp) = make_uint2(w0, w1);
    }
  }
}

// f32 VALU kernel: one workgroup per (position, kv head, batch row); wave w owns heads w, w+4, ...
// Both products accumulate in f64 and round once to f32 (the exactly rounded dot products up to one
// f64 rounding), and the softmax's exponentials and sum are evaluated in f64 and rounded once: two
// f32 evaluation orders differ by more than the fp32 parity bar at the model level, the exactly
// rounded result is the one every order approximates.
template <int D>
__global__ __launch_bounds__(256) void prefill_f32_kernel(G4PrefillArgs a, int t_alloc) {
  extern __shared__ float smem[];  // [4 waves][t_alloc] scores
  const int S = a.seq, H = a.kv_heads, R = a.group;
  const int pos = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t bh = (int64_t)b * H + h;
  const uint8_t* km = a.key_mask + (int64_t)b * a.key_mask_stride;
  const float* kbase = reinterpret_cast<const float*>(a.k) + bh * a.k_stride * D;
  const float* vbase = reinterpret_cast<const float*>(a.vt) + bh * D * a.k_stride;
  float* sc = smem + w * t_alloc;
  const int kmin = a.window > 0 ? max(0, pos - a.window + 1) : 0;
  for (int r = w; r < R; r += 4) {
    const float* qrow = reinterpret_cast<const float*>(a.q) + ((((int64_t)b * S + pos) * H + h) * R + r) * D;
    float mx = kF32Min;
    for (int key = kmin + lane; key <= pos; key += 64) {
      double acc = 0.0;
      for (int d = 0; d < D; ++d) acc = fma((double)qrow[d], (double)kbase[kt_index(key, d, D)], acc);
      const float s = km[key] ? (float)acc : kF32Min;
      sc[key - kmin] = s;
      mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    double l64 = 0.0;  // the softmax sum in f64 of the f32 exponentials, rounded once
    for (int key = kmin + lane; key <= pos; key += 64) l64 += (double)exp_f32_exact(sc[key - kmin] - mx);
    for (int m = 32; m >= 1; m >>= 1) l64 += __shfl_xor(l64, m, 64);
    const float l = (float)l64;
    const bool masked = mx == kF32Min;
    const int k0 = masked ? 0 : kmin, k1 = masked ? S - 1 : pos;
    const float lt = masked ? (float)S : l;
    float* orow = reinterpret_cast<float*>(a.out) + ((((int64_t)b * S + pos) * H + h) * R + r) * D;
    for (int d = lane; d < D; d += 64) {
      double o = 0.0;
      for (int key = k0; key <= k1; ++key) {
        const float p = masked ? 1.0f / lt : exp_f32_exact(sc[key - kmin] - mx) / lt;
        o = fma((double)p, (double)vbase[vt_index(key, d, D)], o);
      }
      orow[d] = (float)o;
    }
  }
}

#include "g4_prefill_lds.h"

constexpr int kLdsBytes = 160 * 1024;  // gfx950 LDS per workgroup

// Two waves per SIMD, two 16-row column blocks each (measured per 32-key chunk against one wave per
// SIMD with three or four blocks, which reuse each LDS tile more but leave a lone wave to overlap
// its own MFMA, LDS and vector work: 1.85 ms vs 2.04 / 2.66 ms for the config-4 global layer).
constexpr int kPfBlocks = 2;  // 16-row column blocks per wave
constexpr int kPfWaves = 8;   // waves per workgroup

// Largest key-mask row (bytes) the LDS-staged kernel of head dim 128 / 256 can hold next to its
// static tile buffers on each device; 0 when the limit could not be raised. Written once per device
// by setup_prefill_kernels (under device_setup's std::call_once), read after it.
int g_lds_max_seq[kMaxDevices][2];

template <int D>
int raise_prefill_lds_limit(int device) {
  int& max_seq = g_lds_max_seq[device][D == 256];
  max_seq = 0;
  hipFuncAttributes attr;
  // a failed query or limit leaves max_seq at 0: every row then takes the register kernel
  if (hipFuncGetAttributes(&attr, (const void*)prefill_bf16_lds_kernel<D, kPfBlocks, kPfWaves>) != hipSuccess) {
    (void)hipGetLastError();
    return G4_OK;
  }
  const int room = (kLdsBytes - (int)attr.sharedSizeBytes) / 16 * 16;
  const int cap = room < kPfMaxSeq ? room : kPfMaxSeq;
  if (cap > 0 && raise_lds_limit(device, (const void*)prefill_bf16_lds_kernel<D, kPfBlocks, kPfWaves>, cap))
    max_seq = cap;
  return G4_OK;
}

template <int D>
void launch_prefill_lds(const G4PrefillArgs& a, hipStream_t st) {
  const int ppb = kPfWaves * kPfBlocks * (16 / a.group);
  const dim3 grid((unsigned)((a.seq + ppb - 1) / ppb) * (unsigned)a.kv_heads * (unsigned)a.batch);
  const size_t lds = ((size_t)a.seq + 15) / 16 * 16;
  hipLaunchKernelGGL((prefill_bf16_lds_kernel<D, kPfBlocks, kPfWaves>), grid, dim3(kPfWaves * 64), lds, st, a);
}

}  // namespace

int setup_prefill_kernels(int device) {
  const int rc = raise_prefill_lds_limit<128>(device);
  return rc != G4_OK ? rc : raise_prefill_lds_limit<256>(device);
}

}  // namespace g4

extern "C" int g4_prefill_attention(const G4PrefillArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_prefill_attention: args is NULL");
  const G4PrefillArgs& a = *args;
  if (a.dtype != G4_DTYPE_F32 && a.dtype != G4_DTYPE_BF16)
    return fail(G4_ERR_INVALID, "g4_prefill_attention: dtype %d", a.dtype);
  if (a.batch <= 0 || a.seq <= 0 || a.kv_heads <= 0 || a.group <= 0)
    return fail(G4_ERR_INVALID, "g4_prefill_attention: batch/seq/kv_heads/group must be positive");
  if (!supported_head_dim(a.head_dim)) return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: head_dim %d", a.head_dim);
  if (a.k_stride < a.seq || a.k_stride % 64)
    return fail(G4_ERR_INVALID, "g4_prefill_attention: k_stride %d (need >= seq, multiple of 64)", a.k_stride);
  if (a.window < 0) return fail(G4_ERR_INVALID, "g4_prefill_attention: window %d", a.window);
  if (!a.q || !a.k || !a.vt || !a.out || !a.key_mask || a.key_mask_stride < a.seq)
    return fail(G4_ERR_INVALID, "g4_prefill_attention: NULL pointer or key_mask_stride < seq");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a.dtype == G4_DTYPE_BF16) {
    if (16 % a.group) return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: bf16 needs group dividing 16");
    if (a.head_dim < 32)
      return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: bf16 head_dim %d (bf16 prefill covers 32..512)",
                  a.head_dim);
    int dev = 0;
    const int rc = device_setup(&dev);
    if (rc != G4_OK) return rc;
    // head dims 128/256: K/V chunks staged through LDS, when the row's key mask fits next to them
    if (a.head_dim == 256 && a.seq <= g_lds_max_seq[dev][1]) {
      launch_prefill_lds<256>(a, st);
      return check_launch("g4_prefill_attention");
    }
    if (a.head_dim == 128 && a.seq <= g_lds_max_seq[dev][0]) {
      launch_prefill_lds<128>(a, st);
      return check_launch("g4_prefill_attention");
    }
    const int rows_per_block = kPrefillWaves * (16 / a.group);
    const dim3 grid((unsigned)((a.seq + rows_per_block - 1) / rows_per_block), a.kv_heads, a.batch);
    const dim3 block(kPrefillWaves * 64);
    switch (a.head_dim) {
      case 32: hipLaunchKernelGGL(prefill_bf16_kernel<32>, grid, block, 0, st, a); break;
      case 64: hipLaunchKernelGGL(prefill_bf16_kernel<64>, grid, block, 0, st, a); break;
      case 128: hipLaunchKernelGGL(prefill_bf16_kernel<128>, grid, block, 0, st, a); break;
      case 256: hipLaunchKernelGGL(prefill_bf16_kernel<256>, grid, block, 0, st, a); break;
      case 512: hipLaunchKernelGGL(prefill_bf16_kernel<512>, grid, block, 0, st, a); break;
      default: return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: bf16 head_dim %d", a.head_dim);
    }
  } else {
    const int t_alloc = a.window > 0 ? (a.window < a.seq ? a.window : a.seq) : a.seq;
    const size_t lds = (size_t)4 * t_alloc * 4;
    if (lds > 64 * 1024) return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: f32 key range %d too long", t_alloc);
    const dim3 grid((unsigned)a.seq, a.kv_heads, a.batch);
    switch (a.head_dim) {
      case 8: hipLaunchKernelGGL(prefill_f32_kernel<8>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 16: hipLaunchKernelGGL(prefill_f32_kernel<16>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 32: hipLaunchKernelGGL(prefill_f32_kernel<32>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 64: hipLaunchKernelGGL(prefill_f32_kernel<64>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 128: hipLaunchKernelGGL(prefill_f32_kernel<128>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 256: hipLaunchKernelGGL(prefill_f32_kernel<256>, grid, dim3(256), lds, st, a, t_alloc); break;
      case 512: hipLaunchKernelGGL(prefill_f32_kernel<512>, grid, dim3(256), lds, st, a, t_alloc); break;
      default: return fail(G4_ERR_UNSUPPORTED, "g4_prefill_attention: head_dim %d", a.head_dim);
    }
  }
  return check_launch("g4_prefill_attention");
}
