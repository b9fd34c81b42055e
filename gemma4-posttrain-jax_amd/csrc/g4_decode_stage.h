// bf16 decode attention for rows of at most 512 slots (the sliding-window ring) with
// D / NSPLIT = 128 value dims per workgroup; included by g4_decode.hip after g4_decode_fast.h.
//
// Requests: q (straight into MFMA operand registers), the key-mask bytes and two 32-slot K
// chunks per wave (registers) go out first, with V^T chunks 0..10 of the workgroup's slice DMA'd
// into LDS (buffer_load ... lds); chunks 11..15 are queued after the softmax's second barrier
// (config 2: 15.39-15.48 us with 8 + 8 chunks, 15.14-15.17 with 10 + 6, 15.09-15.10 with 11 + 5,
// 15.27-15.35 with 12 + 4: each chunk requested early adds to the K loads' contention, each one
// requested late to the tail after the softmax). Wave w stages the tiles of its own 16-row d-block, each tile
// lane-ordered so that it is read back as that lane's MFMA operand. The split keeps the memory
// queue busy through the scores and the softmax without making the barriers wait for the whole
// V issue (a wave blocked on a full queue reaches no barrier), and the value MFMAs of the first
// half run while the second half lands. The barriers wait only for LDS traffic (a
// __syncthreads() fence would also wait for the DMA, which writes LDS); each wave waits for its
// own DMA right before the value MFMAs that read it (the two halves are separate LDS arrays, so
// the compiler's wait for the first does not include the second). The value MFMAs accumulate the
// even chunks in one register set and the odd ones in another, whatever the split.
//
// The appended token: the wave that scores the chunk holding the slot stages the new K row in
// LDS for itself (no barrier) and substitutes it into that chunk's K operand registers; every
// wave writes the new V value into its own staged tile once its DMA has landed and stores the
// patched 16-byte pieces to the cache. The K row is written last (after every load of the
// workgroup).
//
// The softmax runs on all 512 threads: thread t owns 4 consecutive (head, slot) entries of the
// [R][512] score array, so no lanes sit idle behind the R <= 16 MFMA columns.

constexpr int kStageSlots = 2 * NW * 32;  // slots per row handled here (16 chunks)
// LDS row stride of the score/probability array: 64 bytes of padding put the rows of heads
// 0..3 on different banks for the 16-byte MFMA-operand accesses (lane (grp, col) -> row col).
constexpr int kStageStride = kStageSlots + 32;

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr int kVtEarly = 11;                // V^T chunks requested with K (the rest after the softmax)
constexpr int kVtLate = 2 * NW - kVtEarly;
template <int N>
using VtTiles = unsigned char[NW][N][1024];  // [wave][chunk][lane*16]

// The body takes every LDS region as a restrict pointer: once inlined, the compiler knows that the
// score / statistics accesses never touch the tiles the V^T DMA writes, so it does not make them
// wait for that DMA.
template <int D, int NSPLIT>
__device__ __forceinline__ void stage_body(const G4DecodeArgs& a, VtTiles<kVtEarly>* __restrict__ vt_lo_p,
                                           VtTiles<kVtLate>* __restrict__ vt_hi_p, uint16_t* __restrict__ nk_lds,
                                           uint16_t* __restrict__ sp, float* __restrict__ wmax,
                                           float* __restrict__ bsum) {
  VtTiles<kVtEarly>& vt_lo = *vt_lo_p;
  VtTiles<kVtLate>& vt_hi = *vt_hi_p;
  const int R = a.group;

  const int npairs = a.batch * a.kv_heads;
  int pair, h;
  if (NSPLIT == 1) {
    pair = blockIdx.x;
    h = 0;
  } else {  // the two workgroups of a pair share blockIdx.x mod 8, i.e. one XCD
    pair = (int)(blockIdx.x >> 4) * 8 + (int)(blockIdx.x & 7);
    h = (int)(blockIdx.x >> 3) & 1;
  }
  if (pair >= npairs) return;  // padding workgroups of the NSPLIT = 2 grid (whole workgroup)
  const int b = pair / a.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int db = h * NW + w;  // this wave's d-block: value dims [16*db, 16*db + 16)
  const KeyRange kr = key_range(a, b);
  const uint32_t pair_bytes = (uint32_t)a.slot_stride * D * 2u;
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D, pair_bytes);
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride, pair_bytes);
  const int n_chunks = (kr.n_keys + 31) >> 5;  // <= 2*NW: capacity <= 512 is checked on the host
  const bool has_new = kr.new_slot >= 0;
  const bool owner = has_new && (int)((kr.new_slot >> 5) & (NW - 1)) == w;  // scores the appended slot's chunk

  // ---- requests: small rows, q operands, mask bytes, K, then the V^T slice into LDS -------------
  u32x4 nkv = {0u, 0u, 0u, 0u};
  if (owner && lane < D / 8) nkv = load16(reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D + 8 * lane);
  uint32_t nvb = 0;  // new V value of this lane's d row (16*db + col)
  if (has_new) nvb = reinterpret_cast<const uint16_t*>(a.new_v)[(int64_t)pair * D + 16 * db + col];
  bf16x8 qop[D / 32];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)pair * R + (col < R ? col : 0)) * D;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (col < R) v = load16(qrow + 32 * s + 8 * grp);
      qop[s] = as_bf16x8(v);
    }
  }
  const int c0 = w << 5, c1 = (w + NW) << 5;
  uint8_t mb0, mb1;
  const bool ok0 = slot_valid_flat(a, b, kr, c0 + (lane & 31), mb0);
  const bool ok1 = slot_valid_flat(a, b, kr, c1 + (lane & 31), mb1);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 k0[2][D / 32], k1[2][D / 32];
  // a chunk past the row's last one (never scored) re-reads that last chunk: an L2 hit, not HBM
  const int kc_last = n_chunks > 0 ? n_chunks - 1 : 0;
  load_k_chunk<D>(k0, rk, w < n_chunks ? c0 : kc_last << 5, col, grp);
  load_k_chunk<D>(k1, rk, w + NW < n_chunks ? c1 : kc_last << 5, col, grp);
  // Every byte is requested before any compute: a wave stalled on a full memory queue cannot
  // compute anyway, and its K (requested first) has landed by the time its last DMA is queued.
  const uint32_t soff = 256u * db;  // value dims 16 db + col
  // Every wave issues all the DMAs of each part (a chunk past the row's last one re-reads that last
  // chunk, which stays inside the pair's slots), so the compiler knows how many loads are in
  // flight behind each K load and waits for exactly the one it needs.
  const int c_last = n_chunks > 0 ? n_chunks - 1 : 0;
  auto dma_v = [&](auto& tiles, int c, int first) {  // chunk c into tile c - first
    const int cs = c < n_chunks ? c : c_last;
    const uint32_t voff = vt_operand_bytes(4 * cs + grp, col, D);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)&tiles[w][c - first][0],
                                             16, voff, soff, 0, kNonTemporal);
  };
#pragma unroll
  for (int c = 0; c < kVtEarly; ++c) dma_v(vt_lo, c, 0);
  __builtin_amdgcn_sched_barrier(0);
  if (owner && lane < D / 8) reinterpret_cast<u32x4*>(nk_lds)[lane] = nkv;  // read back by this wave only
  const uint64_t vb0 = __ballot(ok0 && mb0 != 0);
  const uint64_t vb1 = __ballot(ok1 && mb1 != 0);

  // ---- scores (each wave: chunks w and w + NW) --------------------------------------------------
  float mx = kBf16Min;
  if (w < n_chunks) {
    patch_k_sel<D>(k0, nk_lds, kr.new_slot, c0, col, grp);
    mx = score_to_lds<D>(k0, qop, vb0, sp, kStageStride, c0, R, col, grp, mx);
  }
  if (w + NW < n_chunks) {
    patch_k_sel<D>(k1, nk_lds, kr.new_slot, c1, col, grp);
    mx = score_to_lds<D>(k1, qop, vb1, sp, kStageStride, c1, R, col, grp, mx);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (grp == 0) wmax[w * 16 + col] = mx;
  wg_barrier();  // scores and wave maxima are in LDS

  // ---- softmax over all threads: thread t owns entries [4t, 4t + 4) of each 2048-entry slice ----
  // (entry e = head * 512 + slot; a wave's 256 entries lie in one head)
  bool all_masked = true;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) all_masked = all_masked && wmax[ww * 16] == kBf16Min;  // per-slot validity
  const int n_scanned = n_chunks << 5;
  const int slot = 256 * (w & 1) + 4 * lane;
  float ev[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // heads 4i + w/2 (R <= 16)
    const int hh = 4 * i + (w >> 1);
    if (hh < R && !all_masked) {
      float m = kBf16Min;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) m = fmaxf(m, wmax[ww * 16 + hh]);
      const uint2 sv = *reinterpret_cast<const uint2*>(sp + hh * kStageStride + slot);
      const float s4[4] = {bf16_lo(sv.x), bf16_hi(sv.x), bf16_lo(sv.y), bf16_hi(sv.y)};
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ev[i][j] = slot + j < n_scanned ? expf(s4[j] - m) : 0.f;
        part += ev[i][j];
      }
      part = wave_sum64(part);
      if (lane == 0) bsum[2 * hh + (w & 1)] = part;
    }
  }
  wg_barrier();  // block sums are in LDS
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = kVtEarly; c < 2 * NW; ++c) dma_v(vt_hi, c, kVtEarly);
  __builtin_amdgcn_sched_barrier(0);
  const float pu = round_bf16(1.0f / (float)a.capacity);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = 4 * i + (w >> 1);
    if (hh < R) {
      float p[4];
      if (all_masked) {  // no valid slot: uniform bf16(1/capacity) over the capacity
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = slot + j < a.capacity ? pu : 0.f;
      } else {
        const float l = bsum[2 * hh] + bsum[2 * hh + 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = ev[i][j] / l;
      }
      const uint2 pw = make_uint2(f32_to_bf16_bits(p[0]) | (f32_to_bf16_bits(p[1]) << 16),
                                  f32_to_bf16_bits(p[2]) | (f32_to_bf16_bits(p[3]) << 16));
      *reinterpret_cast<uint2*>(sp + hh * kStageStride + slot) = pw;
    }
  }
  wg_barrier();  // probabilities are in LDS

  // ---- values: this wave's d-block over every chunk ---------------------------------------------
  // (the compiler waits for a half's DMA before the first LDS access to that half)
  const int cn = (int)(kr.new_slot >> 5), gn = (int)(kr.new_slot & 31) >> 3, en = (int)(kr.new_slot & 7);
  const int n_chunks2 = all_masked ? (a.capacity + 31) >> 5 : n_chunks;
  floatx4 oacc = {0.f, 0.f, 0.f, 0.f}, oacc1 = {0.f, 0.f, 0.f, 0.f};  // even / odd chunks
  auto value_half = [&](auto& tiles, int c_first, auto count) {
    constexpr int N = decltype(count)::value;
    // the appended slot's value into the staged tile (the lanes of the slot's 8-slot group), and that
    // patched 16-byte piece (8 slots of one value dim) into the cache: whole pieces, 256 contiguous
    // bytes per wave, instead of one two-byte value in every 16 bytes of them (configs[1]: 15.20 ->
    // 14.94 us). Only this workgroup reads its dims' pieces, so nothing it still loads can see it.
    if (has_new && cn >= c_first && cn < c_first + N && grp == gn) {
      *reinterpret_cast<uint16_t*>(&tiles[w][cn - c_first][16 * lane + 2 * en]) = (uint16_t)nvb;
      uint16_t* cv = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
      *reinterpret_cast<u32x4*>(cv + vt_index(kr.new_slot & ~(int64_t)7, 16 * db + col, D)) =
          *reinterpret_cast<const u32x4*>(&tiles[w][cn - c_first][16 * lane]);
    }
    u32x4 vt[N];  // every operand read before the MFMA chain (LDS latency paid once)
    bf16x8 pp[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (c_first + i < n_chunks) {
        vt[i] = *reinterpret_cast<const u32x4*>(&tiles[w][i][16 * lane]);
        pp[i] = prob_operand(sp, kStageStride, ((c_first + i) << 5) + 8 * grp, R, col);
      }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {  // even chunks into oacc, odd ones into oacc1
      if (c_first + i < n_chunks) {
        if (((c_first + i) & 1) == 0) oacc = mfma16x16x32(as_bf16x8(vt[i]), pp[i], oacc);
        else oacc1 = mfma16x16x32(as_bf16x8(vt[i]), pp[i], oacc1);
      }
    }
  };
  value_half(vt_lo, 0, std::integral_constant<int, kVtEarly>{});
  value_half(vt_hi, kVtEarly, std::integral_constant<int, kVtLate>{});
  oacc += oacc1;
  for (int c = n_chunks; c < n_chunks2; ++c) {  // fully masked linear row: slots never scanned
    const u32x4 v = buffer_load16(rv, vt_operand_bytes(4 * c + grp, col, D), 256u * db);
    oacc = mfma16x16x32(as_bf16x8(v), prob_operand(sp, kStageStride, (c << 5) + 8 * grp, R, col), oacc);
  }

  // ---- the fused append's K row write (after every cache load of this workgroup) ---------------
  // Workgroup h writes K row elements [h*D/NSPLIT, (h+1)*D/NSPLIT) (its V^T pieces went out with the
  // value MFMAs). The other workgroup of the pair may still read that K row; it substitutes the
  // staged row for it, so what it reads does not matter.
  if (has_new) {
    constexpr int DS = D / NSPLIT;  // K row elements [h*DS, (h+1)*DS): lanes holding 8 of them each
    uint16_t* ck = reinterpret_cast<uint16_t*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D;
    if (owner && lane >= h * DS / 8 && lane < (h + 1) * DS / 8)
      *reinterpret_cast<u32x4*>(ck + kt_index(kr.new_slot, 8 * lane, D)) = nkv;
  }
  // lane (grp, col < R) holds O^T[d = 16*db + 4*grp + j][head col]
  if (col < R) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)pair * R + col) * D;
    const uint32_t w0 = f32_to_bf16_bits(oacc[0]) | (f32_to_bf16_bits(oacc[1]) << 16);
    const uint32_t w1 = f32_to_bf16_bits(oacc[2]) | (f32_to_bf16_bits(oacc[3]) << 16);
    *reinterpret_cast<uint2*>(orow + 16 * db + 4 * grp) = make_uint2(w0, w1);
  }
}

template <int D, int NSPLIT>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_stage_kernel(G4DecodeArgs a) {
  static_assert(D / NSPLIT == 16 * NW, "one 16-row d-block of V^T per wave");
  __shared__ __attribute__((aligned(1024))) VtTiles<kVtEarly> vt_lo;  // chunks 0..10
  __shared__ __attribute__((aligned(1024))) VtTiles<kVtLate> vt_hi;   // chunks 11..15
  __shared__ __attribute__((aligned(16))) uint16_t nk_lds[D];
  extern __shared__ float smem[];
  uint16_t* sp = reinterpret_cast<uint16_t*>(smem);                      // [R][stride] scores, then probabilities
  float* wmax = reinterpret_cast<float*>(sp + a.group * kStageStride);  // [NW][16] wave maxima
  float* bsum = wmax + NW * 16;                                         // [R][2] sums of 256-slot blocks
  stage_body<D, NSPLIT>(a, &vt_lo, &vt_hi, nk_lds, sp, wmax, bsum);
}
