// bf16 decode attention, key-split scores / head-dim-split values; included by g4_decode.hip
// after g4_decode_bf16.h (same namespace and helpers).
//
// Phase 1 splits the slots over the waves (wave w scores chunks w, w+NW, ...; two chunks' K in
// flight per round) and leaves bf16-rounded, masked scores in LDS. Phase 2 splits the head
// dimension instead: wave w owns DPW 16-row d-blocks and runs the value MFMAs over every chunk,
// so it keeps DPW accumulators (not D/16) and no cross-wave reduction of O is needed. Its V^T
// loads are double-buffered in groups of G chunks; the first two groups are issued as soon as
// phase 1's K registers are free, so they overlap the softmax statistics.

template <int D>
struct DsplitShape {
  static constexpr int NDB = D / 16;   // d-blocks
  static constexpr int DPW = NDB / NW; // d-blocks per wave
  static constexpr int G = 8;          // chunks per V group (G * DPW * 4 registers)
  static_assert(DPW >= 1, "needs D >= 16 * waves");
};

template <int D>
__device__ __forceinline__ void load_v_group(u32x4 (&vg)[DsplitShape<D>::G][DsplitShape<D>::DPW],
                                             __amdgpu_buffer_rsrc_t rv, int64_t ss, int g, int n_chunks2, int w,
                                             int col, int grp) {
  using S = DsplitShape<D>;
#pragma unroll
  for (int i = 0; i < S::G; ++i) {
    const int c = g * S::G + i;
    if (c < n_chunks2) {
      const uint32_t voff = (uint32_t)(col * ss + (c << 5) + 8 * grp) * 2u;
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii)
        vg[i][ii] = buffer_load16(rv, voff, (uint32_t)(16 * (w * S::DPW + ii) * ss) * 2u);
    }
  }
}

template <int D>
__device__ __forceinline__ void consume_v_group(u32x4 (&vg)[DsplitShape<D>::G][DsplitShape<D>::DPW],
                                                floatx4 (&oacc)[DsplitShape<D>::DPW], const DecodeLds& L,
                                                int t_alloc, int g, int n_chunks2, int R, int w, int col, int grp,
                                                int64_t new_slot) {
  using S = DsplitShape<D>;
#pragma unroll
  for (int i = 0; i < S::G; ++i) {
    const int c = g * S::G + i;
    if (c < n_chunks2) {
      const int kb = (c << 5) + 8 * grp;
      const bf16x8 pop = prob_operand(L.pl, t_alloc, kb, R, col);
      const int64_t off = new_slot - kb;
#pragma unroll
      for (int ii = 0; ii < S::DPW; ++ii) {
        u32x4 v = vg[i][ii];
        if (off >= 0 && off < 8) {  // the appended slot: value from the staged new V row
          const uint32_t nvb = L.nv[16 * (w * S::DPW + ii) + col];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t word = v[q];
            const uint32_t patched = (off & 1) ? ((word & 0x0000ffffu) | (nvb << 16)) : ((word & 0xffff0000u) | nvb);
            v[q] = q == (int)(off >> 1) ? patched : word;
          }
        }
        oacc[ii] = mfma16x16x32(as_bf16x8(v), pop, oacc[ii]);
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_dsplit_kernel(G4DecodeArgs a, int t_alloc) {
  using S = DsplitShape<D>;
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
  const int n_chunks = (kr.n_keys + 31) >> 5;

  // ---- phase 1 (slots split over waves), first round peeled so the small loads ride behind it ----
  float mx = kBf16Min;
  {
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
    if (w < n_chunks) {
      patch_k<D>(k0, L.nk, kr.new_slot, c0, col, grp);
      score_chunk<D>(k0, L.qs, vb0, L.sc, t_alloc, c0, R, col, grp, mx);
    }
    if (w + NW < n_chunks) {
      patch_k<D>(k1, L.nk, kr.new_slot, c1, col, grp);
      score_chunk<D>(k1, L.qs, vb1, L.sc, t_alloc, c1, R, col, grp, mx);
    }
  }
  for (int c = w + 2 * NW; c < n_chunks; c += 2 * NW) {  // rows longer than 2*NW chunks
    const int c0 = c << 5, c1 = (c + NW) << 5;
    u32x4 k0[2][D / 32], k1[2][D / 32];
    load_k_chunk<D>(k0, rk, c0, col, grp);
    load_k_chunk<D>(k1, rk, c1, col, grp);
    uint8_t mb0, mb1;
    const bool ok0 = slot_valid_flat(a, b, kr, c0 + (lane & 31), mb0);
    const bool ok1 = slot_valid_flat(a, b, kr, c1 + (lane & 31), mb1);
    const uint64_t vb0 = __ballot(ok0 && mb0 != 0);
    const uint64_t vb1 = __ballot(ok1 && mb1 != 0);
    patch_k<D>(k0, L.nk, kr.new_slot, c0, col, grp);
    score_chunk<D>(k0, L.qs, vb0, L.sc, t_alloc, c0, R, col, grp, mx);
    if (c + NW < n_chunks) {
      patch_k<D>(k1, L.nk, kr.new_slot, c1, col, grp);
      score_chunk<D>(k1, L.qs, vb1, L.sc, t_alloc, c1, R, col, grp, mx);
    }
  }

  // ---- phase 2 (head dim split over waves) --------------------------------------------------------
  // The first two V groups are requested before the softmax statistics; a fully masked linear
  // row (uniform weights up to the capacity) can need more chunks than were scored.
  const int n_chunks_all = (a.capacity + 31) >> 5;
  u32x4 va[S::G][S::DPW], vb[S::G][S::DPW];
  __builtin_amdgcn_sched_barrier(0);
  load_v_group<D>(va, rv, a.slot_stride, 0, n_chunks, w, col, grp);
  load_v_group<D>(vb, rv, a.slot_stride, 1, n_chunks, w, col, grp);
  __builtin_amdgcn_sched_barrier(0);
  const Softmax sm = softmax_stats(mx, L.sc, L.wmax, L.wsum, t_alloc, n_chunks, R, w, col, grp);
  const int n_chunks2 = sm.all_masked ? n_chunks_all : n_chunks;
  write_probs(L, t_alloc, n_chunks2 << 5, R, sm.all_masked, round_bf16(1.0f / (float)a.capacity), a.capacity);
  __syncthreads();
  if (n_chunks2 != n_chunks) {  // reload the first groups with the longer uniform range
    load_v_group<D>(va, rv, a.slot_stride, 0, n_chunks2, w, col, grp);
    load_v_group<D>(vb, rv, a.slot_stride, 1, n_chunks2, w, col, grp);
  }
  floatx4 oacc[S::DPW];
#pragma unroll
  for (int ii = 0; ii < S::DPW; ++ii) oacc[ii] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int n_groups = (n_chunks2 + S::G - 1) / S::G;
  for (int g = 0; g < n_groups; g += 2) {
    consume_v_group<D>(va, oacc, L, t_alloc, g, n_chunks2, R, w, col, grp, kr.new_slot);
    if (g + 2 < n_groups) load_v_group<D>(va, rv, a.slot_stride, g + 2, n_chunks2, w, col, grp);
    if (g + 1 < n_groups) consume_v_group<D>(vb, oacc, L, t_alloc, g + 1, n_chunks2, R, w, col, grp, kr.new_slot);
    if (g + 3 < n_groups) load_v_group<D>(vb, rv, a.slot_stride, g + 3, n_chunks2, w, col, grp);
  }

  // lane (grp, col < R) holds O^T[d = 16*(w*DPW + ii) + 4*grp + j][head col]
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
