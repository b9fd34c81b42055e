// One-token GQA decode attention over ring / linear KV caches (g4_decode_attention).
//
// Replaces make_cached_qk_masks + the score/softmax/value einsums of
// gemma4_posttrain_jax/model.py:338-365, 496-499 for S = 1. The reference rounds scores to the
// activation dtype, normalises with an f32 softmax over the whole row and rounds the
// probabilities before the value product; the bf16 kernel reproduces that rounding exactly by
// running the softmax in two phases over scores kept in LDS (max/sum first, then exact
// probabilities for the value pass) instead of an online rescale.
//
// bf16 path: one workgroup (NW waves) per (b, kv head). Each wave takes 32-slot chunks.
//   QK on MFMA 16x16x32: A = 16 key rows (16-byte loads along d), B = the R query heads padded
//   to 16 columns. Key rows are assigned so that lane (grp, col) ends up holding head `col`'s
//   scores for keys c0 + 8*grp + e, e = 0..7 — exactly the B-operand layout of the value MFMA.
//   PV on MFMA 16x16x32: A = V^T rows (16-byte loads along keys from the transposed cache),
//   B = probabilities, accumulators = O^T[d, head].
// f32 path: a VALU kernel with the same two-phase structure (the tiny fp32 configs).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kDecodeWaves = 8;

struct KeyRange {
  int64_t q;         // absolute query position
  int n_keys;        // slots scanned: all Wc ring slots, or 0..min(q, C-1) for a linear cache
  int64_t new_slot;  // slot of the fused append (-1: none)
};

__device__ __forceinline__ KeyRange key_range(const G4DecodeArgs& a, int b) {
  KeyRange kr;
  kr.q = a.q_pos ? (int64_t)a.q_pos[b] : (int64_t)a.q_pos_scalar;
  const bool ring = a.kind == G4_CACHE_RING;
  if (ring) {
    kr.n_keys = a.capacity;
  } else {
    int64_t last = kr.q < (int64_t)a.capacity - 1 ? kr.q : (int64_t)a.capacity - 1;
    kr.n_keys = last < 0 ? 0 : (int)(last + 1);
  }
  if (a.new_k) {
    if (ring) {
      kr.new_slot = floor_mod(kr.q, a.capacity);
    } else {
      int64_t s = kr.q < 0 ? 0 : kr.q;
      kr.new_slot = s > a.capacity - 1 ? a.capacity - 1 : s;
    }
  } else {
    kr.new_slot = -1;
  }
  return kr;
}

// Validity of cache slot `slot` for the query (model.py:352-364).
__device__ __forceinline__ bool key_valid(const G4DecodeArgs& a, int b, const KeyRange& kr, int slot) {
  if (slot >= kr.n_keys) return false;
  int64_t pos;
  if (a.kind == G4_CACHE_RING) {
    pos = ring_slot_position(kr.q, slot, a.capacity);
    if (pos < 0 || pos <= kr.q - a.window) return false;
  } else {
    pos = slot;
  }
  if (pos > kr.q || pos >= a.key_mask_stride) return false;
  return a.key_mask[(int64_t)b * a.key_mask_stride + pos] != 0;
}

// Store this token's prepared K/V row into the cache (the fused append). Nothing in the same
// launch reads these locations back from memory: the attention passes substitute the new values.
template <bool BF16, int D>
__device__ __forceinline__ void fused_append(const G4DecodeArgs& a, int pair, const KeyRange& kr) {
  using T = typename Elem<BF16>::T;
  if (kr.new_slot < 0) return;
  const T* nk = reinterpret_cast<const T*>(a.new_k) + (int64_t)pair * D;
  const T* nv = reinterpret_cast<const T*>(a.new_v) + (int64_t)pair * D;
  T* ck = reinterpret_cast<T*>(a.cache_k_w) + ((int64_t)pair * a.slot_stride + kr.new_slot) * D;
  T* cv = reinterpret_cast<T*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride + kr.new_slot;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    ck[d] = nk[d];
    cv[(int64_t)d * a.slot_stride] = nv[d];
  }
}

// ----------------------------------------------------------------------------------------------
// bf16, MFMA
// ----------------------------------------------------------------------------------------------

template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_kernel(G4DecodeArgs a, int t_alloc) {
  constexpr int NW = kDecodeWaves;
  constexpr int KS = D / 32;  // MFMA k-steps over the head dim
  constexpr int DB = D / 16;  // 16-row blocks of d for the value product
  extern __shared__ float smem[];
  const int R = a.group;
  float* sc = smem;                      // [R][t_alloc] rounded, masked scores
  float* wmax = smem + R * t_alloc;      // [NW][16]
  float* wsum = wmax + NW * 16;          // [NW][16]
  float* red = smem;                     // [NW][R][D] value partials (aliases sc after a barrier)

  const int pair = blockIdx.x;
  const int b = pair / a.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const KeyRange kr = key_range(a, b);
  fused_append<true, D>(a, pair, kr);

  const uint16_t* qh = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)pair * R * D;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
  const uint16_t* newk = kr.new_slot >= 0 ? reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D : nullptr;
  const uint16_t* newv = kr.new_slot >= 0 ? reinterpret_cast<const uint16_t*>(a.new_v) + (int64_t)pair * D : nullptr;

  bf16x8 qop[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (col < R) v = load16(qh + col * D + 32 * s + 8 * grp);
    qop[s] = as_bf16x8(v);
  }

  // ---- phase 1: scores for every scanned slot -------------------------------------------------
  const int n_chunks = (kr.n_keys + 31) >> 5;
  float mx = kBf16Min;
  for (int c = w; c < n_chunks; c += NW) {
    const int c0 = c << 5;
    const bool valid = key_valid(a, b, kr, c0 + (lane & 31));
    const uint64_t vbits = __ballot(valid);
    floatx4 acc[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int kslot = c0 + 8 * (col >> 2) + 4 * bb + (col & 3);
      const uint16_t* kp = (kslot == kr.new_slot) ? newk : kbase + (int64_t)kslot * D;
      u32x4 kv[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) kv[s] = load16(kp + 32 * s + 8 * grp);
      floatx4 acc_b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc_b = mfma16x16x32(as_bf16x8(kv[s]), qop[s], acc_b);
      acc[bb] = acc_b;
    }
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kk = 8 * grp + 4 * bb + j;
        const float s = ((vbits >> kk) & 1ull) ? round_bf16(acc[bb][j]) : kBf16Min;
        if (col < R) sc[col * t_alloc + c0 + kk] = s;
        mx = fmaxf(mx, s);
      }
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (grp == 0) wmax[w * 16 + col] = mx;
  __syncthreads();
  float m = kBf16Min;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) m = fmaxf(m, wmax[ww * 16 + col]);
  const bool all_masked = wmax[0] == kBf16Min && [&] {
    for (int ww = 1; ww < NW; ++ww)
      if (wmax[ww * 16] != kBf16Min) return false;
    return true;
  }();

  float l = 0.f;
  if (col < R) {
    for (int c = w; c < n_chunks; c += NW) {
      const float* sp = sc + col * t_alloc + (c << 5) + 8 * grp;
#pragma unroll
      for (int e = 0; e < 8; ++e) l += expf(sp[e] - m);
    }
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (grp == 0) wsum[w * 16 + col] = l;
  __syncthreads();
  float lsum = 0.f;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) lsum += wsum[ww * 16 + col];

  // ---- phase 2: exact probabilities, value product ---------------------------------------------
  // A row with no valid key is the reference's softmax over all-equal fills: 1/T on every slot.
  const int n_keys2 = all_masked ? a.capacity : kr.n_keys;
  const int n_chunks2 = (n_keys2 + 31) >> 5;
  const float p_uniform = round_bf16(1.0f / (float)a.capacity);
  floatx4 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c = w; c < n_chunks2; c += NW) {
    const int c0 = c << 5;
    const int kb = c0 + 8 * grp;
    u32x4 vv[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) vv[i] = load16(vbase + (int64_t)(16 * i + col) * a.slot_stride + kb);
    uint32_t pw[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t lo = 0, hi = 0;
      if (col < R) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int key = kb + 2 * e2 + h2;
          float p;
          if (all_masked) {
            p = key < a.capacity ? p_uniform : 0.f;
          } else {
            p = round_bf16(expf(sc[col * t_alloc + key] - m) / lsum);
          }
          const uint32_t bits = f32_to_bf16_bits(p);
          if (h2 == 0) lo = bits; else hi = bits;
        }
      }
      pw[e2] = lo | (hi << 16);
    }
    const bf16x8 pop = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
    const int64_t off = kr.new_slot - kb;
    if (off >= 0 && off < 8) {
#pragma unroll
      for (int i = 0; i < DB; ++i) {
        const uint32_t nvb = newv[16 * i + col];
        uint32_t word = vv[i][off >> 1];
        word = (off & 1) ? ((word & 0x0000ffffu) | (nvb << 16)) : ((word & 0xffff0000u) | nvb);
        vv[i][off >> 1] = word;
      }
    }
#pragma unroll
    for (int i = 0; i < DB; ++i) oacc[i] = mfma16x16x32(as_bf16x8(vv[i]), pop, oacc[i]);
  }

  // ---- cross-wave reduction of O^T partials -----------------------------------------------------
  __syncthreads();  // every wave is done with sc before red (aliasing it) is written
  if (col < R) {
#pragma unroll
    for (int i = 0; i < DB; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(w * R + col) * D + 16 * i + 4 * grp + j] = oacc[i][j];
    }
  }
  __syncthreads();
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + (int64_t)pair * R * D;
  for (int idx = tid; idx < R * D; idx += NW * 64) {
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) o += red[ww * R * D + idx];
    out[idx] = (uint16_t)f32_to_bf16_bits(o);
  }
}

// ----------------------------------------------------------------------------------------------
// f32, VALU
// ----------------------------------------------------------------------------------------------

template <int D>
__global__ __launch_bounds__(256) void decode_f32_kernel(G4DecodeArgs a, int t_alloc) {
  extern __shared__ float smem[];
  const int R = a.group;
  float* sc = smem;               // [R][t_alloc]
  float* stats = smem + R * t_alloc;  // [R][2] max, sum
  const int pair = blockIdx.x;
  const int b = pair / a.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const KeyRange kr = key_range(a, b);
  fused_append<false, D>(a, pair, kr);
  const float* qh = reinterpret_cast<const float*>(a.q) + (int64_t)pair * R * D;
  const float* kbase = reinterpret_cast<const float*>(a.cache_k) + (int64_t)pair * a.slot_stride * D;
  const float* vbase = reinterpret_cast<const float*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
  const float* newk = kr.new_slot >= 0 ? reinterpret_cast<const float*>(a.new_k) + (int64_t)pair * D : nullptr;
  const float* newv = kr.new_slot >= 0 ? reinterpret_cast<const float*>(a.new_v) + (int64_t)pair * D : nullptr;

  for (int key = tid; key < kr.n_keys; key += blockDim.x) {
    const bool valid = key_valid(a, b, kr, key);
    const float* kp = key == kr.new_slot ? newk : kbase + (int64_t)key * D;
    for (int r = 0; r < R; ++r) {
      float s = 0.f;
      for (int d = 0; d < D; ++d) s = fmaf(qh[r * D + d], kp[d], s);
      sc[r * t_alloc + key] = valid ? s : kF32Min;
    }
  }
  __syncthreads();
  for (int r = w; r < R; r += blockDim.x / 64) {
    float mx = kF32Min;
    for (int key = lane; key < kr.n_keys; key += 64) mx = fmaxf(mx, sc[r * t_alloc + key]);
    mx = wave_max(mx);
    float l = 0.f;
    for (int key = lane; key < kr.n_keys; key += 64) l += expf(sc[r * t_alloc + key] - mx);
    l = wave_sum(l);
    if (lane == 0) {
      stats[2 * r] = mx;
      stats[2 * r + 1] = l;
    }
  }
  __syncthreads();
  const bool all_masked = stats[0] == kF32Min;
  const int n2 = all_masked ? a.capacity : kr.n_keys;
  float* out = reinterpret_cast<float*>(a.out) + (int64_t)pair * R * D;
  for (int idx = tid; idx < R * D; idx += blockDim.x) {
    const int r = idx / D, d = idx - r * D;
    const float m = stats[2 * r], l = all_masked ? (float)a.capacity : stats[2 * r + 1];
    const float* vrow = vbase + (int64_t)d * a.slot_stride;
    float o = 0.f;
    for (int key = 0; key < n2; ++key) {
      const float p = all_masked ? 1.0f / l : expf(sc[r * t_alloc + key] - m) / l;
      const float v = key == kr.new_slot ? newv[d] : vrow[key];
      o = fmaf(p, v, o);
    }
    out[idx] = o;
  }
}

size_t lds_bytes_bf16(const G4DecodeArgs& a, int t_alloc) {
  const size_t scores = (size_t)a.group * t_alloc * 4 + 2 * kDecodeWaves * 16 * 4;
  const size_t red = (size_t)kDecodeWaves * a.group * a.head_dim * 4;
  return scores > red ? scores : red;
}

constexpr size_t kMaxLds = 64 * 1024;

}  // namespace
}  // namespace g4

extern "C" size_t g4_decode_workspace_size(const G4DecodeArgs* args) {
  (void)args;
  return 0;
}

extern "C" int g4_decode_attention(const G4DecodeArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_decode_attention: args is NULL");
  const G4DecodeArgs& a = *args;
  if (a.dtype != G4_DTYPE_F32 && a.dtype != G4_DTYPE_BF16)
    return fail(G4_ERR_INVALID, "g4_decode_attention: dtype %d", a.dtype);
  if (a.kind != G4_CACHE_LINEAR && a.kind != G4_CACHE_RING)
    return fail(G4_ERR_INVALID, "g4_decode_attention: kind %d", a.kind);
  if (a.batch <= 0 || a.kv_heads <= 0 || a.group <= 0 || a.group > 16)
    return fail(G4_ERR_INVALID, "g4_decode_attention: batch %d kv_heads %d group %d (1..16)", a.batch, a.kv_heads,
                a.group);
  if (!supported_head_dim(a.head_dim)) return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: head_dim %d", a.head_dim);
  if (a.capacity <= 0 || a.slot_stride < a.capacity || a.slot_stride % 64)
    return fail(G4_ERR_INVALID, "g4_decode_attention: capacity %d / slot_stride %d", a.capacity, a.slot_stride);
  if (a.kind == G4_CACHE_RING && a.window <= 0) return fail(G4_ERR_INVALID, "g4_decode_attention: ring needs window > 0");
  if (!a.q || !a.cache_k || !a.cache_vt || !a.out || !a.key_mask)
    return fail(G4_ERR_INVALID, "g4_decode_attention: NULL q/cache/out/key_mask");
  if (a.kind == G4_CACHE_LINEAR && a.key_mask_stride < a.capacity)
    return fail(G4_ERR_INVALID, "g4_decode_attention: key_mask_stride %d < capacity %d", a.key_mask_stride, a.capacity);
  if (a.key_mask_stride <= 0) return fail(G4_ERR_INVALID, "g4_decode_attention: key_mask_stride must be positive");
  if ((a.new_k == nullptr) != (a.new_v == nullptr))
    return fail(G4_ERR_INVALID, "g4_decode_attention: new_k and new_v must be given together");
  if (a.new_k && !a.cache_k_w) return fail(G4_ERR_INVALID, "g4_decode_attention: fused append needs cache_k_w");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int t_alloc = (a.capacity + 31) / 32 * 32;
  const dim3 grid((unsigned)((int64_t)a.batch * a.kv_heads));
  if (a.dtype == G4_DTYPE_BF16) {
    const size_t lds = lds_bytes_bf16(a, t_alloc);
    if (lds > kMaxLds)
      return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: capacity %d x group %d needs %zu B of LDS (> %zu)",
                  a.capacity, a.group, lds, kMaxLds);
    const dim3 block(kDecodeWaves * 64);
    switch (a.head_dim) {
      case 32: hipLaunchKernelGGL(decode_bf16_kernel<32>, grid, block, lds, st, a, t_alloc); break;
      case 64: hipLaunchKernelGGL(decode_bf16_kernel<64>, grid, block, lds, st, a, t_alloc); break;
      case 128: hipLaunchKernelGGL(decode_bf16_kernel<128>, grid, block, lds, st, a, t_alloc); break;
      case 256: hipLaunchKernelGGL(decode_bf16_kernel<256>, grid, block, lds, st, a, t_alloc); break;
      default: return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: bf16 head_dim %d", a.head_dim);
    }
  } else {
    const size_t lds = (size_t)a.group * t_alloc * 4 + (size_t)a.group * 8;
    if (lds > kMaxLds) return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: f32 capacity %d too large", a.capacity);
    const dim3 block(256);
    switch (a.head_dim) {
      case 8: hipLaunchKernelGGL(decode_f32_kernel<8>, grid, block, lds, st, a, t_alloc); break;
      case 16: hipLaunchKernelGGL(decode_f32_kernel<16>, grid, block, lds, st, a, t_alloc); break;
      case 32: hipLaunchKernelGGL(decode_f32_kernel<32>, grid, block, lds, st, a, t_alloc); break;
      case 64: hipLaunchKernelGGL(decode_f32_kernel<64>, grid, block, lds, st, a, t_alloc); break;
      case 128: hipLaunchKernelGGL(decode_f32_kernel<128>, grid, block, lds, st, a, t_alloc); break;
      case 256: hipLaunchKernelGGL(decode_f32_kernel<256>, grid, block, lds, st, a, t_alloc); break;
      case 512: hipLaunchKernelGGL(decode_f32_kernel<512>, grid, block, lds, st, a, t_alloc); break;
      default: return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: head_dim %d", a.head_dim);
    }
  }
  return check_launch("g4_decode_attention");
}
