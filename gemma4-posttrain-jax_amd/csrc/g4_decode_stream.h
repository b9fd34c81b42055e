// bf16 decode attention for rows of at most 16 chunks (512 slots: the sliding-window ring),
// with every byte of the (b, kv head)'s K and V requested up front; included by g4_decode.hip
// after g4_decode_dsplit.h.
//
// The exact softmax needs all scores before any value product, so a plain two-phase kernel
// leaves HBM idle between "all of K" and "all of V". Here the V^T tiles a wave will consume for
// chunks 0..7 are DMA'd straight into LDS (buffer_load ... lds: no registers held) at kernel
// start, next to the K loads; the tiles for chunks 8..15 are loaded into the K registers as soon
// as the first K chunk is scored. Each staged tile is the wave's own MFMA operand in lane order
// (lane l's 16 bytes at tile + 16*l), so it is read back without bank conflicts or barriers.

template <int D>
struct StreamShape {
  static constexpr int DPW = DsplitShape<D>::DPW;  // d-blocks per wave in the value pass
  static constexpr int NA = 8;                     // chunks whose V tiles are staged in LDS
  static constexpr int MAXC = 16;                  // chunks per row handled by this kernel
  static constexpr int TILES_PER_WAVE = NA * DPW;  // 1 KiB tiles per wave in LDS
};

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds_tile, uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_tile, 16, voffset, soffset,
                                           0, 0);
}

template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_stream_kernel(G4DecodeArgs a, int t_alloc) {
  using S = StreamShape<D>;
  extern __shared__ float smem[];
  const int R = a.group;
  const DecodeLds L = carve<D>(smem, R, t_alloc);
  const int pair = blockIdx.x;
  const int b = pair / a.kv_heads;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const KeyRange kr = key_range(a, b);
  const uint32_t pair_bytes = (uint32_t)a.slot_stride * D * 2u;
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D, pair_bytes);
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride, pair_bytes);
  const int64_t ss = a.slot_stride;
  const int n_chunks = (kr.n_keys + 31) >> 5;
  // V tiles in LDS after the other regions, 1 KiB aligned: wave w owns TILES_PER_WAVE tiles
  const uintptr_t va0 = ((uintptr_t)(L.pl + R * t_alloc) + 1023) & ~(uintptr_t)1023;
  char* va = reinterpret_cast<char*>(va0) + w * S::TILES_PER_WAVE * 1024;

  // ---- requests: V tiles of chunks 0..NA-1 -> LDS, both K chunks -> registers --------------------
#pragma unroll
  for (int c = 0; c < S::NA; ++c) {
    if (c < n_chunks) {
      const uint32_t voff = (uint32_t)(col * ss + (c << 5) + 8 * grp) * 2u;
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii)
        dma16(rv, va + (c * S::DPW + ii) * 1024, voff, (uint32_t)(16 * (w * S::DPW + ii) * ss) * 2u);
    }
  }
  const int c0 = w << 5, c1 = (w + NW) << 5;
  u32x4 k0[2][D / 32], k1[2][D / 32];
  load_k_chunk<D>(k0, rk, c0, col, grp);
  load_k_chunk<D>(k1, rk, c1, col, grp);
  uint8_t mb0, mb1;
  const bool ok0 = slot_valid_flat(a, b, kr, c0 + (lane & 31), mb0);
  const bool ok1 = slot_valid_flat(a, b, kr, c1 + (lane & 31), mb1);
  stage_small<D>(a, pair, kr, L, R);
  const uint64_t vb0 = __ballot(ok0 && mb0 != 0);
  const uint64_t vb1 = __ballot(ok1 && mb1 != 0);
  __syncthreads();  // q and the new rows are in LDS

  // ---- scores; the second half of V goes into the first K chunk's registers -----------------------
  float mx = kBf16Min;
  if (w < n_chunks) {
    patch_k<D>(k0, L.nk, kr.new_slot, c0, col, grp);
    score_chunk<D>(k0, L.qs, vb0, L.sc, t_alloc, c0, R, col, grp, mx);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 vbr[S::NA][S::DPW];
#pragma unroll
  for (int c = 0; c < S::NA; ++c) {
    const int cc = S::NA + c;
    if (cc < n_chunks) {
      const uint32_t voff = (uint32_t)(col * ss + (cc << 5) + 8 * grp) * 2u;
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii) vbr[c][ii] = buffer_load16(rv, voff, (uint32_t)(16 * (w * S::DPW + ii) * ss) * 2u);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (w + NW < n_chunks) {
    patch_k<D>(k1, L.nk, kr.new_slot, c1, col, grp);
    score_chunk<D>(k1, L.qs, vb1, L.sc, t_alloc, c1, R, col, grp, mx);
  }
  const Softmax sm = softmax_stats(mx, L.sc, L.wmax, L.wsum, t_alloc, n_chunks, R, w, col, grp);
  const int n_chunks2 = sm.all_masked ? ((a.capacity + 31) >> 5) : n_chunks;
  write_probs(L, t_alloc, n_chunks2 << 5, R, sm.all_masked, round_bf16(1.0f / (float)a.capacity), a.capacity);
  __syncthreads();

  // ---- value pass over this wave's d-blocks --------------------------------------------------------
  // The LDS tiles are the oldest outstanding loads: with every chunk present, at most the
  // NA*DPW register loads above may still be in flight; otherwise drain everything.
  if (n_chunks == S::MAXC) {
    static_assert(S::NA * S::DPW == 16 || S::NA * S::DPW == 8, "wait count below");
    if constexpr (S::NA * S::DPW == 16) __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
  } else {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  floatx4 oacc[S::DPW];
#pragma unroll
  for (int ii = 0; ii < S::DPW; ++ii) oacc[ii] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto pv = [&](u32x4 v, int c, int ii) {
    const int kb = (c << 5) + 8 * grp;
    const int64_t off = kr.new_slot - kb;
    if (off >= 0 && off < 8) {  // the appended slot: value from the staged new V row
      const uint32_t nvb = L.nv[16 * (w * S::DPW + ii) + col];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t word = v[q];
        const uint32_t patched = (off & 1) ? ((word & 0x0000ffffu) | (nvb << 16)) : ((word & 0xffff0000u) | nvb);
        v[q] = q == (int)(off >> 1) ? patched : word;
      }
    }
    oacc[ii] = mfma16x16x32(as_bf16x8(v), prob_operand(L.pl, t_alloc, kb, R, col), oacc[ii]);
  };
#pragma unroll
  for (int c = 0; c < S::NA; ++c) {
    if (c < n_chunks) {
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii)
        pv(*reinterpret_cast<const u32x4*>(va + (c * S::DPW + ii) * 1024 + lane * 16), c, ii);
    }
  }
#pragma unroll
  for (int c = 0; c < S::NA; ++c) {
    if (S::NA + c < n_chunks) {
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii) pv(vbr[c][ii], S::NA + c, ii);
    }
  }
  // fully masked linear row: uniform weights over slots that were never scanned
  for (int c = n_chunks; c < n_chunks2; ++c) {
    const uint32_t voff = (uint32_t)(col * ss + (c << 5) + 8 * grp) * 2u;
#pragma unroll
    for (int ii = 0; ii < S::DPW; ++ii) pv(buffer_load16(rv, voff, (uint32_t)(16 * (w * S::DPW + ii) * ss) * 2u), c, ii);
  }

  store_appended<D>(a, pair, kr, L);
  if (col < R) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)pair * R + col) * D;
#pragma unroll
    for (int ii = 0; ii < S::DPW; ++ii) {
      const uint32_t w0 = f32_to_bf16_bits(oacc[ii][0]) | (f32_to_bf16_bits(oacc[ii][1]) << 16);
      const uint32_t w1 = f32_to_bf16_bits(oacc[ii][2]) | (f32_to_bf16_bits(oacc[ii][3]) << 16);
      *reinterpret_cast<uint2*>(orow + 16 * (w * S::DPW + ii) + 4 * grp) = make_uint2(w0, w1);
    }
  }
}
