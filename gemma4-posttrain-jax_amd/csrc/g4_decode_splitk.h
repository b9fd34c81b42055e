// bf16 decode attention over long rows, split over 512-slot key ranges (flash-decoding style):
// the global-layer linear cache of a long context, where a few (b, kv head) pairs hold tens of
// thousands of slots. Included by g4_decode.hip after g4_decode_stage.h.
//
// Three launches, one workgroup per (pair, split) in the first two:
//   scores   K of the split -> bf16-rounded masked scores (workspace) and, per head, the split's
//            max m_s and l_s = sum exp(s - m_s). Also the fused append: the split holding the
//            appended slot substitutes the new K row and writes the slot (K row and V^T column)
//            back to the cache after its loads.
//   values   V^T loads of the split are issued first, then the split's scores and every split's
//            (m_s, l_s), so that one wait covers them; the row statistics
//            m = max m_s, l = sum_s l_s * exp(m_s - m) are formed (fixed split order), then the
//            exact probabilities bf16(exp(s - m) / l) of the split and its f32 partial of O
//            (configs[2]: 119 -> 116-117 us per step against three dependent round trips).
//   combine  O = sum of the partials in split order, rounded to bf16.
// The probabilities are rounded exactly as the single-pass kernels round them (after the
// division by the full-row sum), so the result differs from theirs only in f32 summation order.
//
// Workspace: scores bf16 [pairs][R][C32] | stats f32 [pairs][splits][R][2] |
//            partials f32 [pairs][splits][R][D]      (C32 = capacity rounded up to 32 * 16).

constexpr int kSplitSlots = 2 * NW * 32;  // slots per split (16 chunks)

struct SplitKWorkspace {
  uint16_t* scores;
  float* stats;
  float* partials;
  int n_splits;  // splits per pair: ceil(capacity / kSplitSlots)
  int c_pad;     // row length of the score array: n_splits * kSplitSlots
};

__host__ __device__ inline size_t splitk_workspace_bytes(int npairs, int R, int D, int capacity) {
  const size_t n_splits = (size_t)(capacity + kSplitSlots - 1) / kSplitSlots;
  return (size_t)npairs * R * n_splits * kSplitSlots * 2 + (size_t)npairs * n_splits * R * 2 * 4 +
         (size_t)npairs * n_splits * R * D * 4;
}

__device__ __forceinline__ bf16x8 q_operand_global(const G4DecodeArgs& a, int pair, int R, int D, int col, int grp,
                                                   int s) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (col < R)
    v = load16(reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)pair * R + col) * D + 32 * s + 8 * grp);
  return as_bf16x8(v);
}

// From D = 256 the q rows sit in LDS (read one 32-dim slice at a time) and a wave holds one K chunk
// at a time (its second chunk is loaded into the first one's registers after that is scored): 96
// registers at D = 256, so two workgroups share a CU and one's loads overlap the other's scoring
// and statistics (configs[2]: 130.5 -> 117.6 us per step; with both chunks and q in registers, 206
// registers and one workgroup per CU).
template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) __attribute__((amdgpu_waves_per_eu(D == 256 ? 4 : 1))) void
decode_bf16_splitk_scores_kernel(G4DecodeArgs a,
                                                                                       SplitKWorkspace ws) {
  __shared__ __attribute__((aligned(16))) uint16_t nk_lds[D];
  // D >= 256: the q rows [R][D] in LDS, read one 32-dim slice at a time (register budget)
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[D > 128 ? 16 * D : 1];
  extern __shared__ float smem[];
  const int R = a.group;
  uint16_t* sp = reinterpret_cast<uint16_t*>(smem);                // [R][stride] scores of the split
  float* wmax = reinterpret_cast<float*>(sp + R * kStageStride);  // [NW][16]
  float* bsum = wmax + NW * 16;                                    // [R][2]
  const int pair = blockIdx.x / ws.n_splits, split = blockIdx.x % ws.n_splits;
  const int b = pair / a.kv_heads;
  const KeyRange kr = key_range(a, b);
  const int n_chunks = (kr.n_keys + 31) >> 5;
  const int cbase = split * 2 * NW;  // first chunk of the split
  if (cbase >= n_chunks) return;     // the split lies beyond the row (whole workgroup)
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D,
                (uint32_t)a.slot_stride * D * 2u);
  const bool has_new = kr.new_slot >= 0 && (kr.new_slot >> 5) >= cbase && (kr.new_slot >> 5) < cbase + 2 * NW;
  const bool owner = has_new && (int)((kr.new_slot >> 5) & (NW - 1)) == w;

  u32x4 nkv = {0u, 0u, 0u, 0u};
  if (owner && lane < D / 8) nkv = load16(reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D + 8 * lane);
  bf16x8 qop[D / 32];
  u32x4 qv[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};  // D >= 256: thread t's q pieces t, t + 512
  const uint16_t* qg = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)pair * R * D;
  if constexpr (D <= 128) {
#pragma unroll
    for (int s = 0; s < D / 32; ++s) qop[s] = q_operand_global(a, pair, R, D, col, grp, s);
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (tid + 512 * j < R * D / 8) qv[j] = load16(qg + 8 * (tid + 512 * j));
  }
  const int cc0 = cbase + w, cc1 = cbase + w + NW;  // this wave's chunks
  const int c0 = cc0 << 5, c1 = cc1 << 5;
  uint8_t mb0, mb1;
  const bool ok0 = slot_valid_flat(a, b, kr, c0 + (lane & 31), mb0);
  const bool ok1 = slot_valid_flat(a, b, kr, c1 + (lane & 31), mb1);
  __builtin_amdgcn_sched_barrier(0);
  // both chunks' K in registers at once at D = 128; from D = 256 the second chunk is loaded into the
  // first one's registers after they are scored
  constexpr bool kBothChunks = D <= 128;
  u32x4 k0[2][D / 32], k1[2][D / 32];
  load_k_chunk<D, true>(k0, rk, c0, col, grp);
  if constexpr (kBothChunks) load_k_chunk<D, true>(k1, rk, c1, col, grp);
  __builtin_amdgcn_sched_barrier(0);
  if (owner && lane < D / 8) reinterpret_cast<u32x4*>(nk_lds)[lane] = nkv;  // read back by this wave only
  const uint64_t vb0 = __ballot(ok0 && mb0 != 0);
  const uint64_t vb1 = __ballot(ok1 && mb1 != 0);
  if constexpr (D > 128) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (tid + 512 * j < R * D / 8) reinterpret_cast<u32x4*>(q_lds)[tid + 512 * j] = qv[j];
    __syncthreads();  // q rows in LDS
  }
  auto score = [&](const u32x4(&kv)[2][D / 32], uint64_t vbits, int local, float m) {
    if constexpr (D <= 128)
      return score_to_lds<D>(kv, qop, vbits, sp, kStageStride, local, R, col, grp, m);
    else
      return score_to_lds_qlds<D>(kv, q_lds, vbits, sp, kStageStride, local, R, col, grp, m);
  };

  // scores of the split at local slots [0, 512): chunk cc at local offset 32 * (cc - cbase)
  float mx = kBf16Min;
  if (cc0 < n_chunks) {
    patch_k_sel<D>(k0, nk_lds, kr.new_slot, c0, col, grp);
    mx = score(k0, vb0, 32 * w, mx);
  }
  if constexpr (!kBothChunks) {
    if (cc1 < n_chunks) load_k_chunk<D, true>(k0, rk, c1, col, grp);
  }
  u32x4(&kc1)[2][D / 32] = kBothChunks ? k1 : k0;
  if (cc1 < n_chunks) {
    patch_k_sel<D>(kc1, nk_lds, kr.new_slot, c1, col, grp);
    mx = score(kc1, vb1, 32 * (w + NW), mx);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (grp == 0) wmax[w * 16 + col] = mx;
  __syncthreads();

  // split statistics on all threads (thread t: local slots 256*(w&1) + 4*lane .. +3 of head 4i + w/2)
  const int n_local = (n_chunks - cbase < 2 * NW ? n_chunks - cbase : 2 * NW) << 5;  // slots scored here
  const int slot = 256 * (w & 1) + 4 * lane;
  float msplit[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = 4 * i + (w >> 1);
    msplit[i] = kBf16Min;
    if (hh < R) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) msplit[i] = fmaxf(msplit[i], wmax[ww * 16 + hh]);
      const uint2 sv = *reinterpret_cast<const uint2*>(sp + hh * kStageStride + slot);
      const float s4[4] = {bf16_lo(sv.x), bf16_hi(sv.x), bf16_lo(sv.y), bf16_hi(sv.y)};
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) part += slot + j < n_local ? expf(s4[j] - msplit[i]) : 0.f;
      part = wave_sum64(part);
      if (lane == 0) bsum[2 * hh + (w & 1)] = part;
      // the split's scores to the workspace (slots beyond n_local are never read)
      *reinterpret_cast<uint2*>(ws.scores + ((int64_t)pair * R + hh) * ws.c_pad + split * kSplitSlots + slot) = sv;
    }
  }
  __syncthreads();
  if (tid < R) {
    float m = kBf16Min;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) m = fmaxf(m, wmax[ww * 16 + tid]);
    float* st = ws.stats + (((int64_t)pair * ws.n_splits + split) * R + tid) * 2;
    st[0] = m;
    st[1] = bsum[2 * tid] + bsum[2 * tid + 1];
  }

  // the fused append's cache write, after this workgroup's loads; the values launch (next in
  // stream order) reads the V^T column from the cache
  if (has_new) {
    uint16_t* ck = reinterpret_cast<uint16_t*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D;
    if (owner && lane < D / 8) *reinterpret_cast<u32x4*>(ck + kt_index(kr.new_slot, 8 * lane, D)) = nkv;
    uint16_t* cv = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
    const uint16_t* nv = reinterpret_cast<const uint16_t*>(a.new_v) + (int64_t)pair * D;
    for (int d = tid; d < D; d += blockDim.x) cv[vt_index(kr.new_slot, d, D)] = nv[d];
  }
}

// Row statistics from the per-split ones (fixed split order): m, l per head into LDS; returns
// whether the row has no valid slot. One pass over the statistics: the (m_s, l_s) pairs of the
// first 256 splits stay in registers between the max and the sum (no second round trip).
__device__ __forceinline__ bool splitk_row_stats(const SplitKWorkspace& ws, int pair, int R, int n_splits_row,
                                                  float* mh, float* lh, int w, int n_waves, int lane) {
  const float* st = ws.stats + (int64_t)pair * ws.n_splits * R * 2;
  for (int hh = w; hh < R; hh += n_waves) {  // one wave per head
    float2 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = lane + 64 * j;
      v[j] = s < n_splits_row ? *reinterpret_cast<const float2*>(st + (s * R + hh) * 2) : make_float2(kBf16Min, 0.f);
    }
    float m = kBf16Min;
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, v[j].x);
    for (int s = lane + 256; s < n_splits_row; s += 64) m = fmaxf(m, st[(s * R + hh) * 2]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    // l = sum_s l_s * exp(m_s - m), per lane in split order, then across lanes in a fixed tree
    float l = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lane + 64 * j < n_splits_row) l += v[j].y * expf(v[j].x - m);
    for (int s = lane + 256; s < n_splits_row; s += 64) l += st[(s * R + hh) * 2 + 1] * expf(st[(s * R + hh) * 2] - m);
    l = wave_sum64(l);
    if (lane == 0) {
      mh[hh] = m;
      lh[hh] = l;
    }
  }
  __syncthreads();
  return mh[0] == kBf16Min;  // head 0's max (key validity does not depend on the head)
}

template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_splitk_values_kernel(G4DecodeArgs a,
                                                                                       SplitKWorkspace ws) {
  // DSPLIT workgroups per (pair, split), one 16-row d-block per wave each: V^T takes 64 registers
  // per lane, so two workgroups fit on a CU and one's loads overlap the other's tail.
  constexpr int DSPLIT = D / 16 / NW;
  constexpr int DPW = 1;
  static_assert(DSPLIT >= 1 && DSPLIT * NW * 16 == D, "whole d-blocks per wave");
  __shared__ float mh[16], lh[16];
  extern __shared__ float smem[];
  const int R = a.group;
  uint16_t* sp = reinterpret_cast<uint16_t*>(smem);  // [R][stride] probabilities of the split
  int item, dh;  // both value halves of a (pair, split) on one XCD
  xcd_item_part((int)blockIdx.x, a.batch * a.kv_heads * ws.n_splits, DSPLIT, item, dh);
  const int pair = item / ws.n_splits, split = item % ws.n_splits;
  const int b = pair / a.kv_heads;
  const KeyRange kr = key_range(a, b);
  const int n_chunks = (kr.n_keys + 31) >> 5;
  const int n_splits_row = (n_chunks + 2 * NW - 1) / (2 * NW);
  const int cbase = split * 2 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride,
                (uint32_t)a.slot_stride * D * 2u);
  const int n_chunks_cap = (a.capacity + 31) >> 5;
  if (cbase >= n_chunks_cap) return;  // beyond the capacity (whole workgroup)

  // V^T of the split's scanned chunks, requested before anything else
  const int n_here = cbase < n_chunks ? (n_chunks - cbase < 2 * NW ? n_chunks - cbase : 2 * NW) : 0;
  u32x4 vv[2 * NW][DPW];
#pragma unroll
  for (int i = 0; i < 2 * NW; ++i) {
    if (i < n_here) {
      const uint32_t voff = vt_operand_bytes(4 * (cbase + i) + grp, col, D);
#pragma unroll
      for (int ii = 0; ii < DPW; ++ii) vv[i][ii] = buffer_load16_nt(rv, voff, 256u * ((dh * NW + w) * DPW + ii));
    }
  }
  // this thread's scores of the split (4 slots of up to 4 heads), requested with the statistics so
  // that one wait covers both
  const int slot = 256 * (w & 1) + 4 * lane;
  uint2 svh[4] = {{0u, 0u}, {0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = 4 * i + (w >> 1);
    if (hh < R && n_here > 0)
      svh[i] = *reinterpret_cast<const uint2*>(ws.scores + ((int64_t)pair * R + hh) * ws.c_pad + split * kSplitSlots + slot);
  }
  __builtin_amdgcn_sched_barrier(0);
  const bool all_masked = splitk_row_stats(ws, pair, R, n_splits_row, mh, lh, w, NW, lane);
  if (!all_masked && split >= n_splits_row) return;  // nothing of the row here (whole workgroup)
  // a row without any valid slot: uniform bf16(1/capacity) over every slot below the capacity
  const int n_mine = all_masked ? (n_chunks_cap - cbase < 2 * NW ? n_chunks_cap - cbase : 2 * NW) : n_here;
  const float pu = round_bf16(1.0f / (float)a.capacity);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = 4 * i + (w >> 1);
    if (hh < R) {
      float p[4];
      const int gslot = split * kSplitSlots + slot;  // row slot of entry j = 0
      if (all_masked) {
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = gslot + j < a.capacity ? pu : 0.f;
      } else {
        const uint2 sv = svh[i];
        const float s4[4] = {bf16_lo(sv.x), bf16_hi(sv.x), bf16_lo(sv.y), bf16_hi(sv.y)};
        const float m = mh[hh], l = lh[hh];
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = slot + j < (n_here << 5) ? expf(s4[j] - m) / l : 0.f;
      }
      *reinterpret_cast<uint2*>(sp + hh * kStageStride + slot) =
          make_uint2(f32_to_bf16_bits(p[0]) | (f32_to_bf16_bits(p[1]) << 16),
                     f32_to_bf16_bits(p[2]) | (f32_to_bf16_bits(p[3]) << 16));
    }
  }
  __syncthreads();

  floatx4 oacc[DPW];
#pragma unroll
  for (int ii = 0; ii < DPW; ++ii) oacc[ii] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 2 * NW; ++i) {
    if (i < n_here) {
      const bf16x8 pop = prob_operand(sp, kStageStride, (i << 5) + 8 * grp, R, col);
#pragma unroll
      for (int ii = 0; ii < DPW; ++ii) oacc[ii] = mfma16x16x32(as_bf16x8(vv[i][ii]), pop, oacc[ii]);
    }
  }
  for (int i = n_here; i < n_mine; ++i) {  // fully masked row: slots never scanned
    const uint32_t voff = vt_operand_bytes(4 * (cbase + i) + grp, col, D);
    const bf16x8 pop = prob_operand(sp, kStageStride, (i << 5) + 8 * grp, R, col);
#pragma unroll
    for (int ii = 0; ii < DPW; ++ii)
      oacc[ii] = mfma16x16x32(as_bf16x8(buffer_load16_nt(rv, voff, 256u * ((dh * NW + w) * DPW + ii))), pop, oacc[ii]);
  }
  // lane (grp, col < R) holds O^T[d = 16*(w*DPW + ii) + 4*grp + j][head col]
  if (col < R) {
    float* o = ws.partials + (((int64_t)pair * ws.n_splits + split) * R + col) * D;
#pragma unroll
    for (int ii = 0; ii < DPW; ++ii)
      *reinterpret_cast<floatx4*>(o + 16 * ((dh * NW + w) * DPW + ii) + 4 * grp) = oacc[ii];
  }
}

// O = sum of the split partials (split order), bf16. Workgroup (pair, y) owns outputs
// [256 y, 256 y + 256) of the pair's R x D. The partials of the row's scanned splits (known from
// the key range alone) are requested first, 64 splits per batch, before the statistics that only
// tell whether the row is fully masked (then the unscanned splits below the capacity follow, still
// in split order): one round trip per 64 splits instead of one per 8 behind the statistics' loads.
constexpr int kCombineBatch = 64;

__global__ __launch_bounds__(256) void decode_splitk_combine_kernel(G4DecodeArgs a, SplitKWorkspace ws) {
  __shared__ float mh[16], lh[16];
  const int R = a.group, D = a.head_dim;
  const int pair = blockIdx.x;
  const int b = pair / a.kv_heads;
  const KeyRange kr = key_range(a, b);
  const int n_chunks = (kr.n_keys + 31) >> 5;
  const int n_splits_row = (n_chunks + 2 * NW - 1) / (2 * NW);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int idx = (int)blockIdx.y * 256 + tid;
  const bool out_here = idx < R * D;
  // a thread past the pair's outputs reads output 0's partials (in bounds, never stored)
  const float* part = ws.partials + (int64_t)pair * ws.n_splits * R * D + (out_here ? idx : 0);
  // v[j] = partial of split s + j, clamped to the last split (an L2 hit) where s + j >= n
  auto load_batch = [&](int s, int n, float (&v)[kCombineBatch]) {
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) v[j] = part[(int64_t)(s + j < n ? s + j : n - 1) * R * D];
  };
  auto add_batch = [](float o, int s, int n, const float (&v)[kCombineBatch]) {
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j)
      if (s + j < n) o += v[j];
    return o;
  };
  float v[kCombineBatch];
  if (n_splits_row > 0) load_batch(0, n_splits_row, v);
  const bool all_masked = splitk_row_stats(ws, pair, R, n_splits_row, mh, lh, w, (int)(blockDim.x >> 6), lane);
  const int n = all_masked ? ws.n_splits : n_splits_row;
  if (!out_here) return;
  float o = 0.f;
  int s = 0;
  if (n_splits_row > 0) {
    o = add_batch(o, 0, n_splits_row < kCombineBatch ? n_splits_row : kCombineBatch, v);
    s = n_splits_row < kCombineBatch ? n_splits_row : kCombineBatch;
  }
  for (; s < n; s += kCombineBatch) {
    const int e = n - s < kCombineBatch ? n : s + kCombineBatch;  // splits [s, e) of this batch
    load_batch(s, e, v);
    o = add_batch(o, s, e, v);
  }
  reinterpret_cast<uint16_t*>(a.out)[(int64_t)pair * R * D + idx] = (uint16_t)f32_to_bf16_bits(o);
}
