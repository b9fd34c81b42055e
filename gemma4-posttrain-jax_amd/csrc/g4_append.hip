// Fused q/k/v preparation + KV-cache append (g4_kv_append).
//
// Replaces forward_rms_norm / forward_rotary_embedding on q and k, the unscaled v norm, and
// _update_layer_cache of gemma4_posttrain_jax/model.py:463-491, 368-390 with one launch per
// layer. append_kernel: one workgroup per token (b, s); append_tile_kernel (below): one per 8
// tokens of a row, for prefill-sized bf16 chunks. Each wave takes whole head vectors, with lane l
// owning elements [l*D/64, (l+1)*D/64) so a RoPE partner (d +- D/2) is lane l^32 in the same
// register. K rows go to the head-major key cache, V to the transposed value cache
// (cache_vt[b, h, d, slot]) that the MFMA attention kernels read as contiguous key runs.
#include <initializer_list>

#include "g4_common.h"
#include "g4_internal.h"
#include "g4_prep.h"

namespace g4 {
namespace {

enum VecKind { kQ = 0, kK = 1, kV = 2 };

// VEC: bf16 with D >= 128 and every row aligned to its lane's PER elements (checked on the host):
// each lane's elements move in one access per array instead of one per element.
template <bool BF16, int D, bool VEC = false>
__global__ __launch_bounds__(1024) void append_kernel(G4AppendArgs a) {
  using E = Elem<BF16>;
  using T = typename E::T;
  // D >= 64: lane l owns d in [l*D/64, (l+1)*D/64) and its RoPE partner is lane l^32;
  // D < 64: lane l < D owns d = l and its partner is lane l^(D/2).
  constexpr int PER = D >= 64 ? D / 64 : 1;
  constexpr int PARTNER = D >= 64 ? 32 : D / 2;
  const int lane = threadIdx.x & 63;
  const bool lane_on = D >= 64 || lane < D;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int S = a.seq;
  const int token = blockIdx.x;
  const int b = token / S;
  const int s = token - b * S;
  const int H = a.kv_heads;
  const int R = a.group;
  const int nq = a.q ? H * R : 0;
  const int nvec = nq + (a.k ? 2 * H : 0);

  // Destination slot (model.py:373-390): linear writes at start + s with XLA's
  // dynamic_update_slice start clamp; a ring keeps only the chunk's last Wc tokens.
  const int64_t start = a.write_pos ? (int64_t)a.write_pos[b] : (int64_t)a.write_pos_scalar;
  const int64_t cap = a.capacity;
  int64_t slot;
  bool to_cache;
  if (a.kind == G4_CACHE_RING) {
    const int64_t keep = S < cap ? S : cap;
    to_cache = s >= S - keep;
    slot = floor_mod(start + s, cap);
  } else {
    int64_t st = start < 0 ? 0 : start;
    if (st > cap - S) st = cap - S;
    slot = st + s;
    to_cache = true;
  }

  const int64_t in_base = (int64_t)token * a.in_row_stride;
  const int64_t rope_base = (int64_t)token * D;

  for (int vec = wave; vec < nvec; vec += nwaves) {
    int kind, head, r = 0;
    const T* src;
    if (vec < nq) {
      kind = kQ;
      head = vec / R;
      r = vec - head * R;
      src = reinterpret_cast<const T*>(a.q) + in_base + (int64_t)vec * D;
    } else if (vec < nq + H) {
      kind = kK;
      head = vec - nq;
      src = reinterpret_cast<const T*>(a.k) + in_base + (int64_t)head * D;
    } else {
      kind = kV;
      head = vec - nq - H;
      src = reinterpret_cast<const T*>(a.v) + in_base + (int64_t)head * D;
    }

    const bool norm = (kind == kQ && (a.flags & G4_APPEND_NORM_Q)) || (kind == kK && (a.flags & G4_APPEND_NORM_K)) ||
                      (kind == kV && (a.flags & G4_APPEND_NORM_V));
    const bool rope = (kind == kQ && (a.flags & G4_APPEND_ROPE_Q)) || (kind == kK && (a.flags & G4_APPEND_ROPE_K));
    const T* w = norm ? (kind == kQ ? reinterpret_cast<const T*>(a.q_norm_weight)
                                    : (kind == kK ? reinterpret_cast<const T*>(a.k_norm_weight) : nullptr))
                      : nullptr;
    float x[PER];
    prep_head<BF16, D, VEC>(src, w, norm, rope, a.rope_cos + rope_base, a.rope_sin + rope_base, a.eps, lane, x);

    const int64_t bh = (int64_t)b * H + head;
    if (!lane_on) continue;
    // this lane's PER consecutive elements at p (they never cross a 32-element run of the key layout)
    auto store_run = [&](T* p) {
      if constexpr (VEC) {
        st_bf16<PER>(reinterpret_cast<uint16_t*>(p), x);
      } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) E::store(p, e, x[e]);
      }
    };
    auto store_row = [&](T* dst) { store_run(dst + lane * PER); };
    if (kind == kQ) {
      store_row(reinterpret_cast<T*>(a.q_out) + ((((int64_t)token) * H + head) * R + r) * D);
    } else if (kind == kK) {
      if (to_cache) store_run(reinterpret_cast<T*>(a.cache_k) + bh * a.slot_stride * D + kt_index(slot, lane * PER, D));
      if (a.k_out) store_run(reinterpret_cast<T*>(a.k_out) + bh * a.chunk_stride * D + kt_index(s, lane * PER, D));
    } else {
      if (to_cache) {
        T* dst = reinterpret_cast<T*>(a.cache_vt) + bh * D * a.slot_stride;
#pragma unroll
        for (int e = 0; e < PER; ++e) E::store(dst, vt_index(slot, lane * PER + e, D), x[e]);
      }
      if (a.vt_out) {
        T* dst = reinterpret_cast<T*>(a.vt_out) + bh * D * a.chunk_stride;
#pragma unroll
        for (int e = 0; e < PER; ++e) E::store(dst, vt_index(s, lane * PER + e, D), x[e]);
      }
    }
  }
}

// Prefill-sized appends (bf16, the vectorized rows, S >= 8): one 8-wave workgroup per 8
// consecutive tokens of a row, one head vector per wave at a time, at 8 waves per SIMD (the
// prepared vector and its loads take under 64 registers; D = 512 runs at 4). The value cache groups
// 8 slots per 16-byte piece (cache_vt[b, h, slot / 8, d, slot % 8]), so one token's V row is D
// two-byte pieces spread over D / 8 cache lines; when the 8 tokens land in one aligned 8-slot group
// (a cache start and ring size that are multiples of 8) their V rows are staged in LDS and stored as
// whole 16-byte pieces, 16 D contiguous bytes per head, and the chunk copy (vt_out) likewise. Other
// workgroups store V element by element as append_kernel does. Same arithmetic and destinations as
// append_kernel (E2B prefill shape, B 256 x S 256, D 256: a ring layer with its chunk copy 657 -> 421
// us, a linear layer 494 -> 353 us, q alone 251 -> 232 us).
constexpr int kTileTok = 8;
constexpr int kTileThreads = 512;
constexpr int kTileVtBytes = 32 * 1024;  // LDS for the staged V rows: kv_heads * D * 16 bytes at most

template <int D>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(D >= 512 ? 4 : 8))) void
append_tile_kernel(G4AppendArgs a) {
  using T = uint16_t;
  constexpr int PER = D / 64;
  extern __shared__ __attribute__((aligned(16))) uint16_t vt_lds[];  // [H][D][8]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int S = a.seq, H = a.kv_heads, R = a.group;
  const int ntile = (S + kTileTok - 1) / kTileTok;
  const int b = (int)blockIdx.x / ntile;
  const int s0 = ((int)blockIdx.x - b * ntile) * kTileTok;
  const int n_tok = S - s0 < kTileTok ? S - s0 : kTileTok;
  const int nq = a.q ? H * R : 0;
  const int nvec = nq + (a.k ? 2 * H : 0);

  // destination slot of token s (model.py:373-390), as in append_kernel
  const int64_t start = a.write_pos ? (int64_t)a.write_pos[b] : (int64_t)a.write_pos_scalar;
  const int64_t cap = a.capacity;
  auto slot_of = [&](int s, bool& to_cache) -> int64_t {
    if (a.kind == G4_CACHE_RING) {
      const int64_t keep = S < cap ? S : cap;
      to_cache = s >= S - keep;
      return floor_mod(start + s, cap);
    }
    int64_t st = start < 0 ? 0 : start;
    if (st > cap - S) st = cap - S;
    to_cache = true;
    return st + s;
  };
  bool tc_first, tc_last;
  const int64_t slot_first = slot_of(s0, tc_first);
  const int64_t slot_last = slot_of(s0 + n_tok - 1, tc_last);
  // whole 8-slot groups: 8 tokens, consecutive slots from a multiple of 8, one to_cache value
  // (it only switches from false to true along the chunk)
  const bool grouped = a.k && n_tok == kTileTok && slot_first % 8 == 0 && slot_last == slot_first + 7 &&
                       tc_first == tc_last;

  const int jobs = n_tok * nvec;  // job = (token, head vector), tokens outermost
  for (int job = wave; job < jobs; job += nwaves) {
    const int t = job / nvec, vec = job - t * nvec;
    const int s = s0 + t;
    const int64_t in_base = ((int64_t)b * S + s) * a.in_row_stride;
    int kind, head, r = 0;
    const T* src;
    if (vec < nq) {
      kind = kQ;
      head = vec / R;
      r = vec - head * R;
      src = reinterpret_cast<const T*>(a.q) + in_base + (int64_t)vec * D;
    } else if (vec < nq + H) {
      kind = kK;
      head = vec - nq;
      src = reinterpret_cast<const T*>(a.k) + in_base + (int64_t)head * D;
    } else {
      kind = kV;
      head = vec - nq - H;
      src = reinterpret_cast<const T*>(a.v) + in_base + (int64_t)head * D;
    }
    const bool norm = (kind == kQ && (a.flags & G4_APPEND_NORM_Q)) || (kind == kK && (a.flags & G4_APPEND_NORM_K)) ||
                      (kind == kV && (a.flags & G4_APPEND_NORM_V));
    const bool rope = (kind == kQ && (a.flags & G4_APPEND_ROPE_Q)) || (kind == kK && (a.flags & G4_APPEND_ROPE_K));
    const T* w = norm ? (kind == kQ ? reinterpret_cast<const T*>(a.q_norm_weight)
                                    : (kind == kK ? reinterpret_cast<const T*>(a.k_norm_weight) : nullptr))
                      : nullptr;
    const int64_t rope_base = ((int64_t)b * S + s) * D;
    float x[PER];
    prep_head<true, D, true>(src, w, norm, rope, a.rope_cos + rope_base, a.rope_sin + rope_base, a.eps, lane, x);
    const int64_t bh = (int64_t)b * H + head;
    if (kind == kQ) {
      st_bf16<PER>(reinterpret_cast<T*>(a.q_out) + ((((int64_t)b * S + s) * H + head) * R + r) * D + lane * PER, x);
      continue;
    }
    bool to_cache;
    const int64_t slot = slot_of(s, to_cache);
    if (kind == kK) {
      if (to_cache) st_bf16<PER>(reinterpret_cast<T*>(a.cache_k) + bh * a.slot_stride * D + kt_index(slot, lane * PER, D), x);
      if (a.k_out) st_bf16<PER>(reinterpret_cast<T*>(a.k_out) + bh * a.chunk_stride * D + kt_index(s, lane * PER, D), x);
    } else if (grouped) {
#pragma unroll
      for (int e = 0; e < PER; ++e) vt_lds[((int64_t)head * D + lane * PER + e) * 8 + t] = (uint16_t)f32_to_bf16_bits(x[e]);
    } else {
      if (to_cache) {
        T* dst = reinterpret_cast<T*>(a.cache_vt) + bh * D * a.slot_stride;
#pragma unroll
        for (int e = 0; e < PER; ++e) dst[vt_index(slot, lane * PER + e, D)] = (uint16_t)f32_to_bf16_bits(x[e]);
      }
      if (a.vt_out) {
        T* dst = reinterpret_cast<T*>(a.vt_out) + bh * D * a.chunk_stride;
#pragma unroll
        for (int e = 0; e < PER; ++e) dst[vt_index(s, lane * PER + e, D)] = (uint16_t)f32_to_bf16_bits(x[e]);
      }
    }
  }
  if (!grouped) return;  // uniform over the workgroup
  __syncthreads();
  // piece (head, d): the 8 tokens' values of dim d, 16 bytes at slot group slot_first / 8
  for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
    const int hh = i / D, d = i - hh * D;
    const u32x4 piece = reinterpret_cast<const u32x4*>(vt_lds)[i];
    const int64_t bh = (int64_t)b * H + hh;
    if (tc_first)
      *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.cache_vt) + bh * D * a.slot_stride + vt_index(slot_first, d, D)) = piece;
    if (a.vt_out)
      *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.vt_out) + bh * D * a.chunk_stride + vt_index(s0, d, D)) = piece;
  }
}

// The vectorized path needs every row start aligned to one lane's D/64 bf16 elements (and the
// f32 RoPE rows to 16 bytes).
bool vec_rows_ok(const G4AppendArgs& a) {
  const uintptr_t al = (uintptr_t)(a.head_dim / 64) * 2;
  for (const void* p : std::initializer_list<const void*>{a.q, a.k, a.v, a.q_out, a.cache_k, a.k_out,
                                                        a.q_norm_weight, a.k_norm_weight})
    if (reinterpret_cast<uintptr_t>(p) % al) return false;
  for (const void* p : std::initializer_list<const void*>{a.rope_cos, a.rope_sin})
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  return (a.in_row_stride * 2) % (int64_t)al == 0;
}

template <bool BF16>
int launch_append(const G4AppendArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.seq));
  // one wave per head vector (q heads, k heads, v heads) up to 16 waves; more vectors loop
  const int nvec = (a.q ? a.kv_heads * a.group : 0) + (a.k ? 2 * a.kv_heads : 0);
  const dim3 block((unsigned)(64 * (nvec < 1 ? 1 : (nvec > 16 ? 16 : nvec))));
  if (BF16 && a.head_dim >= 128 && vec_rows_ok(a)) {
    const size_t vt_bytes = a.k ? (size_t)a.kv_heads * a.head_dim * 16 : 0;
    // prefill-sized: 8 tokens per workgroup (its 16-byte V stores need 16-byte aligned value arrays)
    const bool vt_aligned = reinterpret_cast<uintptr_t>(a.cache_vt) % 16 == 0 && reinterpret_cast<uintptr_t>(a.vt_out) % 16 == 0;
    if (a.seq >= kTileTok && vt_bytes <= (size_t)kTileVtBytes && vt_aligned) {
      const dim3 tgrid((unsigned)((int64_t)a.batch * ((a.seq + kTileTok - 1) / kTileTok)));
      switch (a.head_dim) {
        case 128: hipLaunchKernelGGL((append_tile_kernel<128>), tgrid, dim3(kTileThreads), vt_bytes, st, a); break;
        case 256: hipLaunchKernelGGL((append_tile_kernel<256>), tgrid, dim3(kTileThreads), vt_bytes, st, a); break;
        case 512: hipLaunchKernelGGL((append_tile_kernel<512>), tgrid, dim3(kTileThreads), vt_bytes, st, a); break;
        default: return fail(G4_ERR_UNSUPPORTED, "g4_kv_append: head_dim %d", a.head_dim);
      }
      return check_launch("g4_kv_append");
    }
    switch (a.head_dim) {
      case 128: hipLaunchKernelGGL((append_kernel<true, 128, true>), grid, block, 0, st, a); break;
      case 256: hipLaunchKernelGGL((append_kernel<true, 256, true>), grid, block, 0, st, a); break;
      case 512: hipLaunchKernelGGL((append_kernel<true, 512, true>), grid, block, 0, st, a); break;
      default: return fail(G4_ERR_UNSUPPORTED, "g4_kv_append: head_dim %d", a.head_dim);
    }
    return check_launch("g4_kv_append");
  }
  switch (a.head_dim) {
    case 8: hipLaunchKernelGGL((append_kernel<BF16, 8>), grid, block, 0, st, a); break;
    case 16: hipLaunchKernelGGL((append_kernel<BF16, 16>), grid, block, 0, st, a); break;
    case 32: hipLaunchKernelGGL((append_kernel<BF16, 32>), grid, block, 0, st, a); break;
    case 64: hipLaunchKernelGGL((append_kernel<BF16, 64>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((append_kernel<BF16, 128>), grid, block, 0, st, a); break;
    case 256: hipLaunchKernelGGL((append_kernel<BF16, 256>), grid, block, 0, st, a); break;
    case 512: hipLaunchKernelGGL((append_kernel<BF16, 512>), grid, block, 0, st, a); break;
    default: return fail(G4_ERR_UNSUPPORTED, "g4_kv_append: head_dim %d", a.head_dim);
  }
  return check_launch("g4_kv_append");
}

}  // namespace
}  // namespace g4

extern "C" int g4_kv_append(const G4AppendArgs* args, void* stream) {
  using g4::fail;
  if (!args) return fail(G4_ERR_INVALID, "g4_kv_append: args is NULL");
  const G4AppendArgs& a = *args;
  if (a.dtype != G4_DTYPE_F32 && a.dtype != G4_DTYPE_BF16) return fail(G4_ERR_INVALID, "g4_kv_append: dtype %d", a.dtype);
  if (a.kind != G4_CACHE_LINEAR && a.kind != G4_CACHE_RING) return fail(G4_ERR_INVALID, "g4_kv_append: kind %d", a.kind);
  if (a.batch <= 0 || a.seq <= 0 || a.kv_heads <= 0)
    return fail(G4_ERR_INVALID, "g4_kv_append: batch/seq/kv_heads must be positive (%d, %d, %d)", a.batch, a.seq,
                a.kv_heads);
  if (!g4::supported_head_dim(a.head_dim)) return fail(G4_ERR_UNSUPPORTED, "g4_kv_append: head_dim %d", a.head_dim);
  if (a.capacity <= 0 || a.slot_stride < a.capacity || a.slot_stride % 64)
    return fail(G4_ERR_INVALID, "g4_kv_append: capacity %d / slot_stride %d (need stride >= capacity, multiple of 64)",
                a.capacity, a.slot_stride);
  if (a.kind == G4_CACHE_LINEAR && a.seq > a.capacity)
    return fail(G4_ERR_INVALID, "g4_kv_append: %d tokens do not fit a linear cache of %d slots", a.seq, a.capacity);
  if (a.k || a.v) {
    if (!a.k || !a.v || !a.cache_k || !a.cache_vt)
      return fail(G4_ERR_INVALID, "g4_kv_append: k/v/cache pointer is NULL");
  } else if (!a.q) {
    return fail(G4_ERR_INVALID, "g4_kv_append: nothing to do (q, k and v are NULL)");
  }
  if (a.in_row_stride < (int64_t)a.kv_heads * a.head_dim)
    return fail(G4_ERR_INVALID, "g4_kv_append: in_row_stride %lld too small", (long long)a.in_row_stride);
  if (a.q) {
    if (a.group <= 0 || !a.q_out) return fail(G4_ERR_INVALID, "g4_kv_append: q needs group > 0 and q_out");
  }
  if ((a.flags & (G4_APPEND_ROPE_K | G4_APPEND_ROPE_Q)) && (!a.rope_cos || !a.rope_sin))
    return fail(G4_ERR_INVALID, "g4_kv_append: RoPE flags need rope_cos/rope_sin");
  if ((a.flags & G4_APPEND_NORM_K) && !a.k_norm_weight) return fail(G4_ERR_INVALID, "g4_kv_append: NORM_K needs k_norm_weight");
  if ((a.flags & G4_APPEND_NORM_Q) && a.q && !a.q_norm_weight)
    return fail(G4_ERR_INVALID, "g4_kv_append: NORM_Q needs q_norm_weight");
  if ((a.k_out || a.vt_out) && (a.chunk_stride < a.seq || a.chunk_stride % 64))
    return fail(G4_ERR_INVALID, "g4_kv_append: chunk_stride %d (need >= seq, multiple of 64)", a.chunk_stride);
  if ((int64_t)a.batch * a.seq > 0x7fffffffLL) return fail(G4_ERR_UNSUPPORTED, "g4_kv_append: too many tokens");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return a.dtype == G4_DTYPE_BF16 ? g4::launch_append<true>(a, st) : g4::launch_append<false>(a, st);
}
