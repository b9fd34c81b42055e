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
#include <type_traits>

#include "g4_common.h"
#include "g4_internal.h"
#include "g4_prep.h"

namespace g4 {
namespace {

constexpr int kDecodeWaves = 8;

struct KeyRange {
  int64_t q;         // absolute query position
  int n_keys;        // slots scanned: ring slots 0..min(q, Wc-1), or 0..min(q, C-1) for a linear cache
  int64_t new_slot;  // slot of the fused append (-1: none)
};

// Slot the token at position q is appended to: q mod Wc for a ring, q clamped to [0, C-1] for a
// linear cache (model.py:373-390).
__device__ __forceinline__ int64_t append_slot(const G4DecodeArgs& a, int64_t q) {
  if (a.kind == G4_CACHE_RING) return floor_mod(q, a.capacity);
  const int64_t s = q < 0 ? 0 : q;
  return s > a.capacity - 1 ? a.capacity - 1 : s;
}

__device__ __forceinline__ KeyRange key_range(const G4DecodeArgs& a, int b) {
  KeyRange kr;
  kr.q = a.q_pos ? (int64_t)a.q_pos[b] : (int64_t)a.q_pos_scalar;
  const bool ring = a.kind == G4_CACHE_RING;
  if (ring) {
    // Before the ring wraps (q < Wc - 1) a slot r > q holds p = r - Wc < 0: never written, never
    // valid (model.py:355-364), so the scan stops at slot q as for a linear cache.
    kr.n_keys = kr.q < (int64_t)a.capacity - 1 ? (kr.q < 0 ? 0 : (int)(kr.q + 1)) : a.capacity;
  } else {
    int64_t last = kr.q < (int64_t)a.capacity - 1 ? kr.q : (int64_t)a.capacity - 1;
    kr.n_keys = last < 0 ? 0 : (int)(last + 1);
  }
  kr.new_slot = a.new_k ? append_slot(a, kr.q) : -1;
  return kr;
}

// (item, part) of workgroup i in a grid of n_items x parts workgroups (an item: a (b, kv head)
// pair, or a (pair, key split)). Workgroups are dealt to the 8 XCDs round robin (i mod 8). With
// n_items a multiple of 8, workgroup i takes item 8 ((i / 8) / parts) + i mod 8 and part
// (i / 8) mod parts: every part of an item runs on one XCD, so what the parts share (score rows,
// statistics, q) is fetched into one L2, and consecutive items still go to consecutive XCDs
// (E2B decode step, two-launch attention: 4.617 -> 4.489 ms). Otherwise item i / parts, part
// i mod parts.
__device__ __forceinline__ void xcd_item_part(int i, int n_items, int parts, int& item, int& part) {
  if (n_items % 8 == 0) {
    const int j = i >> 3;
    part = j % parts;
    item = (j / parts) * 8 + (i & 7);
  } else {
    item = i / parts;
    part = i % parts;
  }
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
  T* ck = reinterpret_cast<T*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D;
  T* cv = reinterpret_cast<T*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    ck[kt_index(kr.new_slot, d, D)] = nk[d];
    cv[vt_index(kr.new_slot, d, D)] = nv[d];
  }
}

#include "g4_decode_bf16.h"
#include "g4_decode_fast.h"
#include "g4_decode_stage.h"
#include "g4_decode_splitk.h"
#include "g4_decode_twopass.h"

// ----------------------------------------------------------------------------------------------
// f32, VALU. Both products accumulate in f64 and round once to f32 (the exactly rounded dot
// products up to one f64 rounding), and the softmax's exponentials and sum are evaluated in f64
// and rounded once, as the f32 prefill kernel does.
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
    for (int r = 0; r < R; ++r) {
      double s = 0.0;
      for (int d = 0; d < D; ++d)
        s = fma((double)qh[r * D + d], (double)(key == kr.new_slot ? newk[d] : kbase[kt_index(key, d, D)]), s);
      sc[r * t_alloc + key] = valid ? (float)s : kF32Min;
    }
  }
  __syncthreads();
  for (int r = w; r < R; r += blockDim.x / 64) {
    float mx = kF32Min;
    for (int key = lane; key < kr.n_keys; key += 64) mx = fmaxf(mx, sc[r * t_alloc + key]);
    mx = wave_max(mx);
    double l = 0.0;  // the softmax sum in f64 of the f32 exponentials, rounded once
    for (int key = lane; key < kr.n_keys; key += 64) l += (double)exp_f32_exact(sc[r * t_alloc + key] - mx);
    for (int m = 32; m >= 1; m >>= 1) l += __shfl_xor(l, m, 64);
    if (lane == 0) {
      stats[2 * r] = mx;
      stats[2 * r + 1] = (float)l;
    }
  }
  __syncthreads();
  const bool all_masked = stats[0] == kF32Min;
  const int n2 = all_masked ? a.capacity : kr.n_keys;
  float* out = reinterpret_cast<float*>(a.out) + (int64_t)pair * R * D;
  for (int idx = tid; idx < R * D; idx += blockDim.x) {
    const int r = idx / D, d = idx - r * D;
    const float m = stats[2 * r], l = all_masked ? (float)a.capacity : stats[2 * r + 1];
    double o = 0.0;
    for (int key = 0; key < n2; ++key) {
      const float p = all_masked ? 1.0f / l : exp_f32_exact(sc[r * t_alloc + key] - m) / l;
      const float v = key == kr.new_slot ? newv[d] : vbase[vt_index(key, d, D)];
      o = fma((double)p, (double)v, o);
    }
    out[idx] = (float)o;
  }
}

// LDS: scores f32 | wave max/sum | q bf16 | new K, V rows bf16 | probabilities bf16, and for the
// key-split kernel (head dims below 128) the O partials [NW][R][D] f32 aliasing from 0.
size_t lds_bytes_bf16(const G4DecodeArgs& a, int t_alloc, bool with_partials) {
  const size_t scores = (size_t)a.group * t_alloc * 4 + 2 * kDecodeWaves * 16 * 4 + (size_t)a.group * a.head_dim * 2 +
                        (size_t)2 * a.head_dim * 2 + (size_t)a.group * t_alloc * 2;
  const size_t red = with_partials ? (size_t)kDecodeWaves * a.group * a.head_dim * 4 : 0;
  return scores > red ? scores : red;
}

constexpr size_t kMaxLds = 64 * 1024;       // default dynamic-LDS limit
constexpr size_t kMaxLdsFast = 160 * 1024;  // gfx950: 160 KiB of LDS per workgroup

// Dynamic LDS of the staged kernel: scores/probabilities bf16 [R][512 + 32] | wave maxima [NW][16] |
// block sums [R][2] (the V^T tiles and the new K row are static).
size_t stage_lds_bytes(int R) { return (size_t)R * kStageStride * 2 + (size_t)kDecodeWaves * 16 * 4 + (size_t)R * 2 * 4; }

// The set-up's record for kernel `fn` (device_setup first): G4_OK when its raised LDS limit is in
// place, else the error a launch of it returns.
int need_lds_limit(const void* fn, const char* what) {
  int dev = 0;
  const int setup = device_setup(&dev);
  if (setup != G4_OK) return setup;
  if (!lds_limit_raised(dev, fn))
    return fail(G4_ERR_LAUNCH, "g4_decode_attention: the LDS limit of the %s kernel could not be raised on device %d",
                what, dev);
  return G4_OK;
}

template <int D, int NSPLIT>
int launch_stage(const G4DecodeArgs& a, hipStream_t st) {
  const int setup = need_lds_limit((const void*)decode_bf16_stage_kernel<D, NSPLIT>, "ring-stage");
  if (setup != G4_OK) return setup;
  const int64_t npairs = (int64_t)a.batch * a.kv_heads;
  const int64_t blocks = NSPLIT == 1 ? npairs : (npairs + 7) / 8 * 8 * NSPLIT;
  hipLaunchKernelGGL((decode_bf16_stage_kernel<D, NSPLIT>), dim3((unsigned)blocks), dim3(kDecodeWaves * 64),
                     stage_lds_bytes(a.group), st, a);
  return G4_OK;
}

template <int D, int NSPLIT, bool LONG>
int launch_fast(const G4DecodeArgs& a, int t_alloc, size_t lds, hipStream_t st) {
  const int setup = need_lds_limit((const void*)decode_bf16_fast_kernel<D, NSPLIT, LONG>, "long-row");
  if (setup != G4_OK) return setup;
  const int64_t npairs = (int64_t)a.batch * a.kv_heads;
  const int64_t blocks = NSPLIT == 1 ? npairs : (npairs + 7) / 8 * 8 * NSPLIT;
  hipLaunchKernelGGL((decode_bf16_fast_kernel<D, NSPLIT, LONG>), dim3((unsigned)blocks), dim3(kDecodeWaves * 64), lds, st,
                     a, t_alloc);
  return G4_OK;
}

}  // namespace
}  // namespace g4

namespace g4 {
namespace {

// Whether the call takes the split-K path (bf16, head dims 128/256, rows longer than one split).
bool use_split_keys(const G4DecodeArgs& a) {
  if (a.dtype != G4_DTYPE_BF16 || (a.head_dim != 128 && a.head_dim != 256 && a.head_dim != 512)) return false;
  const int t_alloc = (a.capacity + 31) / 32 * 32;
  if (t_alloc <= kSplitSlots) return false;
  if (a.num_splits == G4_DECODE_SPLIT_KEYS) return true;
  if (a.num_splits != 0) return false;
  if (a.head_dim == 512) return true;  // no one-launch kernel at this head dim (rows beyond the two-launch path's)
  const int64_t npairs = (int64_t)a.batch * a.kv_heads;
  return npairs < 256 || fast_lds_bytes(a.group, a.head_dim, t_alloc) > kMaxLdsFast;
}

template <int D>
int launch_split_keys(const G4DecodeArgs& a, hipStream_t st) {
  int setup = need_lds_limit((const void*)decode_bf16_splitk_scores_kernel<D>, "split-K scores");
  if (setup == G4_OK) setup = need_lds_limit((const void*)decode_bf16_splitk_values_kernel<D>, "split-K values");
  if (setup != G4_OK) return setup;
  const int64_t npairs = (int64_t)a.batch * a.kv_heads;
  SplitKWorkspace ws;
  ws.n_splits = (a.capacity + kSplitSlots - 1) / kSplitSlots;
  ws.c_pad = ws.n_splits * kSplitSlots;
  ws.scores = reinterpret_cast<uint16_t*>(a.workspace);
  ws.stats = reinterpret_cast<float*>(ws.scores + npairs * a.group * ws.c_pad);
  ws.partials = ws.stats + npairs * ws.n_splits * a.group * 2;
  const dim3 grid((unsigned)(npairs * ws.n_splits)), block(kDecodeWaves * 64);
  const size_t lds = stage_lds_bytes(a.group);
  hipLaunchKernelGGL(decode_bf16_splitk_scores_kernel<D>, grid, block, lds, st, a, ws);
  hipLaunchKernelGGL(decode_bf16_splitk_values_kernel<D>, dim3((unsigned)(npairs * ws.n_splits * (D / 16 / kDecodeWaves))),
                     block, lds, st, a, ws);
  hipLaunchKernelGGL(decode_splitk_combine_kernel, dim3((unsigned)npairs, (unsigned)((a.group * a.head_dim + 255) / 256)),
                     dim3(256), 0, st, a, ws);
  return G4_OK;
}

// Pairs from which the automatic choice takes the two-launch path for rows of at most 1024
// slots: with fewer, one workgroup per CU holds a whole row and the one-launch kernels are faster
// (measured: 128 pairs 19.3 vs 22.2 us, 512 pairs 71.8 vs 62.9 us on a 512-slot ring).
constexpr int64_t kTwoPassMinPairs = 256;

bool two_pass_applies(const G4DecodeArgs& a) {
  return a.dtype == G4_DTYPE_BF16 && (a.head_dim == 128 || a.head_dim == 256 || a.head_dim == 512) &&
         a.capacity <= kTpMaxSlots;
}

// Head dim 512 (the reference's default global head dim) has no one-launch kernel: its rows take
// the two-launch path up to 1024 slots and the split-K path beyond, whatever the pair count.
bool use_two_pass(const G4DecodeArgs& a) {
  if (!two_pass_applies(a)) return false;
  if (a.num_splits == G4_DECODE_TWO_PASS || a.prep) return true;  // only this path fuses the preparation
  return a.num_splits == 0 && (a.head_dim == 512 || (int64_t)a.batch * a.kv_heads >= kTwoPassMinPairs);
}

template <int D, int NCH>
void launch_tp_values(const G4DecodeArgs& a, const uint16_t* ws, int row_slots, hipStream_t st) {
  hipLaunchKernelGGL((decode_bf16_tp_values_kernel<D, NCH>), dim3((unsigned)((int64_t)a.batch * a.kv_heads * (D / 16 / tp_waves_v<NCH>()))),
                     dim3(tp_waves_v<NCH>() * 64), (size_t)a.group * tp_lds_stride(NCH) * 2, st, a, ws, row_slots);
}

template <int D>
int launch_two_pass(const G4DecodeArgs& a, hipStream_t st) {
  const int64_t npairs = (int64_t)a.batch * a.kv_heads;
  const int cap_chunks = (a.capacity + 31) / 32;
  const int parts = (cap_chunks + kTpWavesS - 1) / kTpWavesS;
  const int row_slots = twopass_row_slots(a.capacity);
  uint16_t* ws = reinterpret_cast<uint16_t*>(a.workspace);
  if (a.prep)
    hipLaunchKernelGGL((decode_bf16_tp_scores_kernel<D, true>), dim3((unsigned)(npairs * parts)), dim3(kTpWavesS * 64),
                       0, st, a, ws, parts, row_slots, *a.prep);
  else
    hipLaunchKernelGGL((decode_bf16_tp_scores_kernel<D, false>), dim3((unsigned)(npairs * parts)),
                       dim3(kTpWavesS * 64), 0, st, a, ws, parts, row_slots, G4DecodePrep{});
  if (cap_chunks <= 16)
    launch_tp_values<D, 16>(a, ws, row_slots, st);
  else if (cap_chunks <= 24)
    launch_tp_values<D, 24>(a, ws, row_slots, st);
  else
    launch_tp_values<D, 32>(a, ws, row_slots, st);
  return G4_OK;
}

}  // namespace
}  // namespace g4

namespace g4 {

// Scratch of g4_decode_attention_noalloc: the workspace of the two-launch and split-K paths held by
// the library, one copy per device for the life of the process. In host code `scratch` names a
// host-side stand-in, not device memory: kernels get the per-device address that
// hipGetSymbolAddress returns at set-up (g_scratch).
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
void* g_scratch[kMaxDevices];

// Raises the dynamic-LDS limit of every decode kernel launched with more than the 64 KiB default
// and records this device's address of `scratch` (run once per device by device_setup, with the
// device current, before any of them launches on it).
int setup_decode_kernels(int device) {
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) (void)hipGetLastError();
  g_scratch[device] = e == hipSuccess ? ptr : nullptr;  // null: g4_decode_attention_noalloc reports it
  const int stage = (int)stage_lds_bytes(16);
  const struct {
    const void* fn;
    int bytes;
  } kernels[] = {
      {(const void*)decode_bf16_stage_kernel<128, 1>, stage},
      {(const void*)decode_bf16_stage_kernel<256, 2>, stage},
      {(const void*)decode_bf16_fast_kernel<128, 1, true>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_fast_kernel<128, 1, false>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_fast_kernel<256, 2, true>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_fast_kernel<256, 2, false>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_fast_kernel<256, 1, true>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_fast_kernel<256, 1, false>, (int)kMaxLdsFast},
      {(const void*)decode_bf16_splitk_scores_kernel<128>, stage},
      {(const void*)decode_bf16_splitk_scores_kernel<256>, stage},
      {(const void*)decode_bf16_splitk_scores_kernel<512>, stage},
      {(const void*)decode_bf16_splitk_values_kernel<128>, stage},
      {(const void*)decode_bf16_splitk_values_kernel<256>, stage},
      {(const void*)decode_bf16_splitk_values_kernel<512>, stage},
  };
  // a kernel whose limit stays at the default is recorded as such: only its launches fail
  for (const auto& k : kernels) raise_lds_limit(device, k.fn, k.bytes);
  return G4_OK;
}

}  // namespace g4

extern "C" size_t g4_decode_workspace_size(const G4DecodeArgs* args) {
  using namespace g4;
  if (!args) return 0;
  if (use_two_pass(*args)) return twopass_workspace_bytes(args->batch * args->kv_heads, args->group, args->capacity);
  if (!use_split_keys(*args)) return 0;
  return splitk_workspace_bytes(args->batch * args->kv_heads, args->group, args->head_dim, args->capacity);
}

namespace g4 {

// Host-side argument checks of g4_decode_attention (everything but the workspace, whose need
// depends on the path these arguments select).
int validate_decode_args(const G4DecodeArgs& a) {
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
  if (!a.cache_k || !a.cache_vt || !a.out || !a.key_mask)
    return fail(G4_ERR_INVALID, "g4_decode_attention: NULL cache/out/key_mask");
  if (a.kind == G4_CACHE_LINEAR && a.key_mask_stride < a.capacity)
    return fail(G4_ERR_INVALID, "g4_decode_attention: key_mask_stride %d < capacity %d", a.key_mask_stride, a.capacity);
  if (a.key_mask_stride <= 0) return fail(G4_ERR_INVALID, "g4_decode_attention: key_mask_stride must be positive");
  if ((a.new_k == nullptr) != (a.new_v == nullptr))
    return fail(G4_ERR_INVALID, "g4_decode_attention: new_k and new_v must be given together");
  if (a.prep) {
    const G4DecodePrep& p = *a.prep;
    if (!two_pass_applies(a) || a.num_splits == G4_DECODE_SPLIT_KEYS || a.num_splits > 0)
      return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: fused preparation needs the two-launch path (bf16, head_dim "
                  "128/256/512, capacity <= %d, num_splits 0 or G4_DECODE_TWO_PASS)", kTpMaxSlots);
    if (a.new_k || a.new_v) return fail(G4_ERR_INVALID, "g4_decode_attention: prep replaces new_k / new_v");
    if (!p.q_raw || (p.k_raw == nullptr) != (p.v_raw == nullptr) || (p.k_raw && !a.cache_k_w))
      return fail(G4_ERR_INVALID, "g4_decode_attention: prep needs q_raw, k_raw with v_raw, and cache_k_w to append");
    if (p.in_row_stride < (int64_t)a.kv_heads * a.group * a.head_dim)
      return fail(G4_ERR_INVALID, "g4_decode_attention: prep in_row_stride %lld too small", (long long)p.in_row_stride);
    if (((p.flags & G4_APPEND_NORM_Q) && !p.q_norm_weight) || ((p.flags & G4_APPEND_NORM_K) && !p.k_norm_weight) ||
        ((p.flags & (G4_APPEND_ROPE_Q | G4_APPEND_ROPE_K)) && (!p.rope_cos || !p.rope_sin)))
      return fail(G4_ERR_INVALID, "g4_decode_attention: prep flags %d need their weights / rotary tables", p.flags);
    const uintptr_t al = (uintptr_t)(a.head_dim / 64) * 2;
    for (const void* ptr : {p.q_raw, p.k_raw, p.v_raw, p.q_norm_weight, p.k_norm_weight})
      if (reinterpret_cast<uintptr_t>(ptr) % al)
        return fail(G4_ERR_INVALID, "g4_decode_attention: prep rows need %zu-byte alignment", (size_t)al);
    if ((p.in_row_stride * 2) % (int64_t)al || (reinterpret_cast<uintptr_t>(p.rope_cos) % 16) ||
        (reinterpret_cast<uintptr_t>(p.rope_sin) % 16))
      return fail(G4_ERR_INVALID, "g4_decode_attention: prep row stride / rotary tables misaligned");
  } else if (!a.q) {
    return fail(G4_ERR_INVALID, "g4_decode_attention: NULL q");
  }
  if (a.new_k && !a.cache_k_w) return fail(G4_ERR_INVALID, "g4_decode_attention: fused append needs cache_k_w");
  if (a.num_splits < G4_DECODE_TWO_PASS || a.num_splits > 2)
    return fail(G4_ERR_INVALID, "g4_decode_attention: num_splits %d", a.num_splits);
  if (a.num_splits == G4_DECODE_TWO_PASS && !two_pass_applies(a))
    return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: two-pass needs bf16, head_dim 128/256/512, capacity <= %d",
                kTpMaxSlots);
  if (a.dtype == G4_DTYPE_BF16 && a.head_dim == 512 && a.num_splits > 0)
    return fail(G4_ERR_UNSUPPORTED,
                "g4_decode_attention: bf16 head_dim 512 takes num_splits 0, G4_DECODE_TWO_PASS or G4_DECODE_SPLIT_KEYS");
  if (a.dtype == G4_DTYPE_BF16 && a.head_dim < 32)
    return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: bf16 head_dim %d (bf16 decode covers 32..512)", a.head_dim);
  return G4_OK;
}

}  // namespace g4

extern "C" int g4_decode_attention(const G4DecodeArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_decode_attention: args is NULL");
  const G4DecodeArgs& a = *args;
  {
    const int rc = validate_decode_args(a);
    if (rc != G4_OK) return rc;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int t_alloc = (a.capacity + 31) / 32 * 32;
  const dim3 grid((unsigned)((int64_t)a.batch * a.kv_heads));
  if (use_two_pass(a)) {
    const size_t need = twopass_workspace_bytes(a.batch * a.kv_heads, a.group, a.capacity);
    if (!a.workspace || a.workspace_bytes < need)
      return fail(G4_ERR_WORKSPACE, "g4_decode_attention: two-pass needs %zu B of workspace (have %zu)", need,
                  a.workspace ? a.workspace_bytes : (size_t)0);
    const int rc = a.head_dim == 512   ? launch_two_pass<512>(a, st)
                   : a.head_dim == 256 ? launch_two_pass<256>(a, st)
                                       : launch_two_pass<128>(a, st);
    if (rc != G4_OK) return rc;
    return check_launch("g4_decode_attention");
  }
  if (use_split_keys(a)) {
    const size_t need = splitk_workspace_bytes(a.batch * a.kv_heads, a.group, a.head_dim, a.capacity);
    if (!a.workspace || a.workspace_bytes < need)
      return fail(G4_ERR_WORKSPACE, "g4_decode_attention: split-K needs %zu B of workspace (have %zu)", need,
                  a.workspace ? a.workspace_bytes : (size_t)0);
    const int rc = a.head_dim == 512   ? launch_split_keys<512>(a, st)
                   : a.head_dim == 256 ? launch_split_keys<256>(a, st)
                                       : launch_split_keys<128>(a, st);
    if (rc != G4_OK) return rc;
    return check_launch("g4_decode_attention");
  }
  if (a.num_splits == G4_DECODE_SPLIT_KEYS)
    return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: split-K needs bf16, head_dim 128/256/512, capacity > %d",
                kSplitSlots);
  if (a.dtype == G4_DTYPE_BF16) {
    if (a.head_dim == 128 || a.head_dim == 256) {
      // num_splits: workgroups per (b, kv head), each owning a slice of the value dims
      // (0 = automatic: 2 for head dim 256, else 1)
      const int splits = a.num_splits == 0 ? (a.head_dim == 256 ? 2 : 1) : a.num_splits;
      if (splits != 1 && !(splits == 2 && a.head_dim == 256))
        return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: num_splits %d with head_dim %d", a.num_splits,
                    a.head_dim);
      const size_t lds = fast_lds_bytes(a.group, a.head_dim, t_alloc);
      if (lds > kMaxLdsFast)
        return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: capacity %d x group %d needs %zu B of LDS (> %zu)",
                    a.capacity, a.group, lds, kMaxLdsFast);
      const bool long_rows = t_alloc > 2 * kDecodeWaves * 32;
      int rc;
      if (!long_rows && splits == a.head_dim / 128) {  // V^T slice of 128 dims x 512 slots staged in LDS
        rc = a.head_dim == 128 ? launch_stage<128, 1>(a, st) : launch_stage<256, 2>(a, st);
        if (rc != G4_OK) return rc;
        return check_launch("g4_decode_attention");
      }
      if (a.head_dim == 128)
        rc = long_rows ? launch_fast<128, 1, true>(a, t_alloc, lds, st) : launch_fast<128, 1, false>(a, t_alloc, lds, st);
      else if (splits == 2)
        rc = long_rows ? launch_fast<256, 2, true>(a, t_alloc, lds, st) : launch_fast<256, 2, false>(a, t_alloc, lds, st);
      else
        rc = long_rows ? launch_fast<256, 1, true>(a, t_alloc, lds, st) : launch_fast<256, 1, false>(a, t_alloc, lds, st);
      if (rc != G4_OK) return rc;
      return check_launch("g4_decode_attention");
    }
    // smaller (test) head dims: key-split kernel with a cross-wave reduction of O
    const size_t lds = lds_bytes_bf16(a, t_alloc, true);
    if (lds > kMaxLds)
      return fail(G4_ERR_UNSUPPORTED, "g4_decode_attention: capacity %d x group %d needs %zu B of LDS (> %zu)",
                  a.capacity, a.group, lds, kMaxLds);
    const dim3 block(kDecodeWaves * 64);
    switch (a.head_dim) {
      case 32: hipLaunchKernelGGL(decode_bf16_kernel<32>, grid, block, lds, st, a, t_alloc); break;
      case 64: hipLaunchKernelGGL(decode_bf16_kernel<64>, grid, block, lds, st, a, t_alloc); break;
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

extern "C" int g4_decode_attention_noalloc(const G4DecodeArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_decode_attention_noalloc: args is NULL");
  if (args->workspace || args->workspace_bytes)
    return fail(G4_ERR_INVALID, "g4_decode_attention_noalloc: workspace must be NULL / 0 (the library's scratch is used)");
  {
    const int rc = validate_decode_args(*args);
    if (rc != G4_OK) return rc;
  }
  G4DecodeArgs a = *args;
  const size_t need = g4_decode_workspace_size(&a);
  if (need > kNoAllocScratchBytes)
    return fail(G4_ERR_WORKSPACE,
                "g4_decode_attention_noalloc: the call needs %zu B of scratch, more than the %zu B the library holds "
                "per device; call g4_decode_attention with a workspace",
                need, kNoAllocScratchBytes);
  if (need) {
    int dev = 0;
    const int rc = device_setup(&dev);
    if (rc != G4_OK) return rc;
    if (!g_scratch[dev])
      return fail(G4_ERR_LAUNCH, "g4_decode_attention_noalloc: the scratch address of device %d is unknown "
                  "(hipGetSymbolAddress failed at set-up)", dev);
    a.workspace = g_scratch[dev];
    a.workspace_bytes = kNoAllocScratchBytes;
  }
  return g4_decode_attention(&a, stream);
}
