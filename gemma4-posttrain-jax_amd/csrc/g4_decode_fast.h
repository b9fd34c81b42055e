// bf16 decode attention for head dims 128 and 256 (the Gemma 4 shapes); included by
// g4_decode.hip after g4_decode_bf16.h (same namespace and helpers).
//
// NSPLIT workgroups of NW waves per (b, kv head); workgroup h owns the value dims
// [h*D/NSPLIT, (h+1)*D/NSPLIT). Every workgroup scores every slot: with NSPLIT = 2 the second
// read of K comes from the XCD's L2, because both workgroups of a pair are placed on one XCD
// (workgroups are dealt to the 8 XCDs round-robin by index). That doubles the CUs with loads in
// flight for the same HBM bytes.
//
// Order of work in a workgroup:
//  1. the small loads (q, the appended K/V row, key-mask bytes) are issued first and the first
//     round of K chunks right behind them, so staging the small rows into LDS waits only for
//     the small loads (gfx9 retires vector loads in issue order);
//  2. each wave scores two 32-slot chunks per round on MFMA with the q operand held in
//     registers; rounded, masked scores go to LDS as bf16 (one 16-byte write per lane);
//  3. once a K chunk is consumed its registers take the V^T loads of 8 chunks (this wave's
//     d-blocks), so V is in flight during the second chunk's scores and the softmax statistics;
//  4. row max and sum across the waves (LDS + two barriers); the exact probabilities
//     bf16(exp(s - m) / l) of each wave's own chunks overwrite its scores in LDS;
//  5. value MFMAs over every chunk for the wave's d-blocks: no cross-wave reduction.

template <int D, int NSPLIT>
struct FastShape {
  static constexpr int NDB = D / 16;               // 16-row d-blocks of V^T
  static constexpr int DPW = NDB / (NW * NSPLIT);  // d-blocks per wave
  static_assert(DPW >= 1 && DPW * NW * NSPLIT == NDB, "head dim must split evenly over the waves");
};

// LDS: q bf16 [R][D] | new K row, new V row bf16 [2][D] | scores, then probabilities,
// bf16 [R][t_alloc] | wave max [NW][16] | wave sum [NW][16] (f32).
struct FastLds {
  uint16_t* qs;
  uint16_t* nk;
  uint16_t* nv;
  uint16_t* sp;
  float* wmax;
  float* wsum;
};

__host__ __device__ constexpr size_t fast_lds_bytes(int R, int D, int t_alloc) {
  return ((size_t)R * D + 2 * (size_t)D + (size_t)R * t_alloc) * 2 + 2 * (size_t)NW * 16 * 4;
}

__device__ __forceinline__ FastLds carve_fast(void* smem, int R, int D, int t_alloc) {
  FastLds l;
  l.qs = reinterpret_cast<uint16_t*>(smem);
  l.nk = l.qs + R * D;
  l.nv = l.nk + D;
  l.sp = l.nv + D;
  l.wmax = reinterpret_cast<float*>(l.sp + R * t_alloc);
  l.wsum = l.wmax + NW * 16;
  return l;
}

// The appended slot's K row comes from the staged new row. The branch is wave-uniform (the one
// chunk holding the slot) and the replacement is a per-lane select, so the K registers are
// updated in place instead of being copied for a divergent branch.
template <int D>
__device__ __forceinline__ void patch_k_sel(u32x4 (&kv)[2][D / 32], const uint16_t* nk, int64_t new_slot, int c0,
                                            int col, int grp) {
  if (new_slot >= c0 && new_slot < c0 + 32) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const bool mine = c0 + 8 * (col >> 2) + 4 * bb + (col & 3) == new_slot;
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        const u32x4 n = *reinterpret_cast<const u32x4*>(nk + 32 * s + 8 * grp);
#pragma unroll
        for (int q = 0; q < 4; ++q) kv[bb][s][q] = mine ? n[q] : kv[bb][s][q];
      }
    }
  }
}

// Scores of one 32-slot chunk (MFMA against the register-held q operand), rounded to bf16 and
// masked; lane (grp, col < R) stores head col's slots c0 + 8*grp .. +7 as one 16-byte word.
template <int D>
__device__ __forceinline__ float score_to_lds(const u32x4 (&kv)[2][D / 32], const bf16x8 (&qop)[D / 32],
                                              uint64_t vbits, uint16_t* sp, int t_alloc, int c0, int R, int col,
                                              int grp, float mx) {
  floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    acc0 = mfma16x16x32(as_bf16x8(kv[0][s]), qop[s], acc0);
    acc1 = mfma16x16x32(as_bf16x8(kv[1][s]), qop[s], acc1);
  }
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k0 = 8 * grp + j, k1 = k0 + 4;
    const float s0 = ((vbits >> k0) & 1ull) ? round_bf16(acc0[j]) : kBf16Min;
    const float s1 = ((vbits >> k1) & 1ull) ? round_bf16(acc1[j]) : kBf16Min;
    mx = fmaxf(mx, fmaxf(s0, s1));
    h[j] = f32_to_bf16_bits(s0);
    h[4 + j] = f32_to_bf16_bits(s1);
  }
  if (col < R) {
    const u32x4 word = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    *reinterpret_cast<u32x4*>(sp + col * t_alloc + c0 + 8 * grp) = word;
  }
  return mx;
}

// score_to_lds with the q operand read from LDS ([R][D] bf16) one 32-dim slice at a time
// (inline-assembly reads, each waited for right before its two MFMAs), so the whole operand is
// never held in registers
template <int D>
__device__ __forceinline__ float score_to_lds_qlds(const u32x4 (&kv)[2][D / 32], const uint16_t* q_lds, uint64_t vbits,
                                                   uint16_t* sp, int t_alloc, int c0, int R, int col, int grp,
                                                   float mx) {
  floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const uint32_t qa = lds_addr(q_lds + (col < R ? col : 0) * D + 8 * grp);
  u32x4 q0 = lds_read16(qa), q1 = lds_read16(qa + 64u);
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    u32x4& q = (s & 1) ? q1 : q0;
    lgkm_wait(s + 1 < D / 32 ? 1 : 0, q);
    if (col >= R) q = u32x4{0u, 0u, 0u, 0u};
    acc0 = mfma16x16x32(as_bf16x8(kv[0][s]), as_bf16x8(q), acc0);
    acc1 = mfma16x16x32(as_bf16x8(kv[1][s]), as_bf16x8(q), acc1);
    if (s + 2 < D / 32) q = lds_read16(qa + 64u * (s + 2));
  }
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k0 = 8 * grp + j, k1 = k0 + 4;
    const float s0 = ((vbits >> k0) & 1ull) ? round_bf16(acc0[j]) : kBf16Min;
    const float s1 = ((vbits >> k1) & 1ull) ? round_bf16(acc1[j]) : kBf16Min;
    mx = fmaxf(mx, fmaxf(s0, s1));
    h[j] = f32_to_bf16_bits(s0);
    h[4 + j] = f32_to_bf16_bits(s1);
  }
  if (col < R) {
    const u32x4 word = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    *reinterpret_cast<u32x4*>(sp + col * t_alloc + c0 + 8 * grp) = word;
  }
  return mx;
}

// V^T operands of chunks [8g, 8g + 8) for d-blocks dblock0 .. dblock0 + DPW - 1.
// (value dims 16 (dblock0 + ii) + col, slots 32 c + 8 grp .. + 7: operand group 4 c + grp)
template <int DPW>
__device__ __forceinline__ void fast_load_v(u32x4 (&vg)[8][DPW], __amdgpu_buffer_rsrc_t rv, int D, int g,
                                            int n_chunks, int dblock0, int col, int grp) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = g * 8 + i;
    if (c < n_chunks) {
      const uint32_t voff = vt_operand_bytes(4 * c + grp, col, D);
#pragma unroll
      for (int ii = 0; ii < DPW; ++ii) vg[i][ii] = buffer_load16_nt(rv, voff, 256u * (dblock0 + ii));
    }
  }
}

// fast_load_v with every load issued (a chunk past the row re-reads the last one), so the
// number of loads behind it is fixed and later waits need not include them
template <int DPW>
__device__ __forceinline__ void fast_load_v_fixed(u32x4 (&vg)[8][DPW], __amdgpu_buffer_rsrc_t rv, int D, int g,
                                                  int n_chunks, int dblock0, int col, int grp) {
  const int c_last = n_chunks > 0 ? n_chunks - 1 : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = g * 8 + i < n_chunks ? g * 8 + i : c_last;
    const uint32_t voff = vt_operand_bytes(4 * c + grp, col, D);
#pragma unroll
    for (int ii = 0; ii < DPW; ++ii) vg[i][ii] = buffer_load16_nt(rv, voff, 256u * (dblock0 + ii));
  }
}

template <int DPW>
__device__ __forceinline__ void fast_consume_v(const u32x4 (&vg)[8][DPW], floatx4 (&oacc)[DPW], const FastLds& L,
                                               int t_alloc, int g, int n_chunks, int R, int dblock0, int col, int grp,
                                               int64_t new_slot) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = g * 8 + i;
    if (c < n_chunks) {
      const int kb = (c << 5) + 8 * grp;
      const bf16x8 pop = prob_operand(L.sp, t_alloc, kb, R, col);
      const int64_t off = new_slot - kb;
#pragma unroll
      for (int ii = 0; ii < DPW; ++ii) {
        u32x4 v = vg[i][ii];
        if (off >= 0 && off < 8) {  // the appended slot: value from the staged new V row
          const uint32_t nvb = L.nv[16 * (dblock0 + ii) + col];
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

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// LONG = false: rows of at most 2*NW chunks (t_alloc <= 512, the sliding-window ring), V requested
// while scoring. LONG = true: any row length, V requested after the scores. Two instantiations
// rather than one kernel with both paths: together they exceed the register file.
template <int D, int NSPLIT, bool LONG>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_fast_kernel(G4DecodeArgs a, int t_alloc) {
  using S = FastShape<D, NSPLIT>;
  extern __shared__ float smem[];
  const int R = a.group;
  const FastLds L = carve_fast(smem, R, D, t_alloc);
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
  const int dblock0 = h * (S::NDB / NSPLIT) + w * S::DPW;
  const KeyRange kr = key_range(a, b);
  const uint32_t pair_bytes = (uint32_t)a.slot_stride * D * 2u;
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D, pair_bytes);
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride, pair_bytes);
  const int n_chunks = (kr.n_keys + 31) >> 5;  // <= 2*NW unless LONG (t_alloc checked on the host)

  // ---- 1. small loads, then the first round of K ------------------------------------------------
  u32x4 qv = {0u, 0u, 0u, 0u}, nkv = {0u, 0u, 0u, 0u}, nvv = {0u, 0u, 0u, 0u};
  const bool has_new = kr.new_slot >= 0;
  if (tid < R * D / 8) qv = load16(reinterpret_cast<const uint16_t*>(a.q) + (int64_t)pair * R * D + 8 * tid);
  if (has_new && tid < D / 8) {
    nkv = load16(reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D + 8 * tid);
    nvv = load16(reinterpret_cast<const uint16_t*>(a.new_v) + (int64_t)pair * D + 8 * tid);
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
  __builtin_amdgcn_sched_barrier(0);
  if (tid < R * D / 8) reinterpret_cast<u32x4*>(L.qs)[tid] = qv;
  if (has_new && tid < D / 8) {
    reinterpret_cast<u32x4*>(L.nk)[tid] = nkv;
    reinterpret_cast<u32x4*>(L.nv)[tid] = nvv;
  }
  const uint64_t vb0 = __ballot(ok0 && mb0 != 0);
  const uint64_t vb1 = __ballot(ok1 && mb1 != 0);
  __syncthreads();  // q and the new rows are in LDS
  bf16x8 qop[D / 32];
#pragma unroll
  for (int s = 0; s < D / 32; ++s) qop[s] = q_operand<D>(L.qs, R, col, grp, s);

  // ---- 2./3. scores; V requested as K registers free up ----------------------------------------
  float mx = kBf16Min;
  u32x4 va[8][S::DPW], vb[8][S::DPW];
  if constexpr (!LONG) {
    if (w < n_chunks) {
      patch_k_sel<D>(k0, L.nk, kr.new_slot, c0, col, grp);
      mx = score_to_lds<D>(k0, qop, vb0, L.sp, t_alloc, c0, R, col, grp, mx);
    }
    __builtin_amdgcn_sched_barrier(0);
    fast_load_v<S::DPW>(va, rv, D, 0, n_chunks, dblock0, col, grp);
    __builtin_amdgcn_sched_barrier(0);
    if (w + NW < n_chunks) {
      patch_k_sel<D>(k1, L.nk, kr.new_slot, c1, col, grp);
      mx = score_to_lds<D>(k1, qop, vb1, L.sp, t_alloc, c1, R, col, grp, mx);
    }
    __builtin_amdgcn_sched_barrier(0);
    fast_load_v<S::DPW>(vb, rv, D, 1, n_chunks, dblock0, col, grp);
    __builtin_amdgcn_sched_barrier(0);
  } else {  // a long row (capacity beyond 2*NW chunks; its filled part may still be shorter)
    if (w < n_chunks) {
      patch_k_sel<D>(k0, L.nk, kr.new_slot, c0, col, grp);
      mx = score_to_lds<D>(k0, qop, vb0, L.sp, t_alloc, c0, R, col, grp, mx);
    }
    if (w + NW < n_chunks) {
      patch_k_sel<D>(k1, L.nk, kr.new_slot, c1, col, grp);
      mx = score_to_lds<D>(k1, qop, vb1, L.sp, t_alloc, c1, R, col, grp, mx);
    }
    for (int c = w + 2 * NW; c < n_chunks; c += 2 * NW) {
      const int e0 = c << 5, e1 = (c + NW) << 5;
      load_k_chunk<D>(k0, rk, e0, col, grp);
      load_k_chunk<D>(k1, rk, e1, col, grp);
      uint8_t m0, m1;
      const bool v0 = slot_valid_flat(a, b, kr, e0 + (lane & 31), m0);
      const bool v1 = slot_valid_flat(a, b, kr, e1 + (lane & 31), m1);
      const uint64_t bits0 = __ballot(v0 && m0 != 0);
      const uint64_t bits1 = __ballot(v1 && m1 != 0);
      patch_k_sel<D>(k0, L.nk, kr.new_slot, e0, col, grp);
      mx = score_to_lds<D>(k0, qop, bits0, L.sp, t_alloc, e0, R, col, grp, mx);
      if (c + NW < n_chunks) {
        patch_k_sel<D>(k1, L.nk, kr.new_slot, e1, col, grp);
        mx = score_to_lds<D>(k1, qop, bits1, L.sp, t_alloc, e1, R, col, grp, mx);
      }
    }
    // V of the first 16 chunks requested now, with the K registers free: it lands while the
    // softmax runs
    __builtin_amdgcn_sched_barrier(0);
    fast_load_v_fixed<S::DPW>(va, rv, D, 0, n_chunks, dblock0, col, grp);
    fast_load_v_fixed<S::DPW>(vb, rv, D, 1, n_chunks, dblock0, col, grp);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- 4. softmax statistics and probabilities --------------------------------------------------
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (grp == 0) L.wmax[w * 16 + col] = mx;
  __syncthreads();
  float m = kBf16Min;
  bool all_masked = true;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) {
    m = fmaxf(m, L.wmax[ww * 16 + col]);
    all_masked = all_masked && L.wmax[ww * 16] == kBf16Min;  // head 0 (key validity is per slot)
  }
  float l = 0.f;
  if (col < R && !all_masked) {
    for (int c = w; c < n_chunks; c += NW) {
      const u32x4 sv = *reinterpret_cast<const u32x4*>(L.sp + col * t_alloc + (c << 5) + 8 * grp);
#pragma unroll
      for (int q = 0; q < 4; ++q) l += expf(bf16_lo(sv[q]) - m) + expf(bf16_hi(sv[q]) - m);
    }
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (grp == 0) L.wsum[w * 16 + col] = l;
  __syncthreads();
  float lt = 0.f;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) lt += L.wsum[ww * 16 + col];
  // a row without any valid slot: uniform bf16(1/capacity) over every slot below the capacity
  const int n_chunks2 = all_masked ? (a.capacity + 31) >> 5 : n_chunks;
  if (col < R) {
    const float pu = round_bf16(1.0f / (float)a.capacity);
    for (int c = w; c < n_chunks2; c += NW) {
      uint16_t* p = L.sp + col * t_alloc + (c << 5) + 8 * grp;
      const u32x4 sv = *reinterpret_cast<const u32x4*>(p);
      u32x4 pw;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float p0, p1;
        if (all_masked) {
          const int k = (c << 5) + 8 * grp + 2 * q;
          p0 = k < a.capacity ? pu : 0.f;
          p1 = k + 1 < a.capacity ? pu : 0.f;
        } else {
          p0 = expf(bf16_lo(sv[q]) - m) / lt;
          p1 = expf(bf16_hi(sv[q]) - m) / lt;
        }
        pw[q] = f32_to_bf16_bits(p0) | (f32_to_bf16_bits(p1) << 16);
      }
      *reinterpret_cast<u32x4*>(p) = pw;
    }
  }
  __syncthreads();

  // ---- 5. value pass over this wave's d-blocks -------------------------------------------------
  if (n_chunks2 != n_chunks) {  // a fully masked row reads V over the whole capacity
    fast_load_v<S::DPW>(va, rv, D, 0, n_chunks2, dblock0, col, grp);
    fast_load_v<S::DPW>(vb, rv, D, 1, n_chunks2, dblock0, col, grp);
  }
  floatx4 oacc[S::DPW];
#pragma unroll
  for (int ii = 0; ii < S::DPW; ++ii) oacc[ii] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int n_groups = (n_chunks2 + 7) / 8;
  for (int g = 0; g < n_groups; g += 2) {
    fast_consume_v<S::DPW>(va, oacc, L, t_alloc, g, n_chunks2, R, dblock0, col, grp, kr.new_slot);
    if (g + 2 < n_groups) fast_load_v<S::DPW>(va, rv, D, g + 2, n_chunks2, dblock0, col, grp);
    if (g + 1 < n_groups)
      fast_consume_v<S::DPW>(vb, oacc, L, t_alloc, g + 1, n_chunks2, R, dblock0, col, grp, kr.new_slot);
    if (g + 3 < n_groups) fast_load_v<S::DPW>(vb, rv, D, g + 3, n_chunks2, dblock0, col, grp);
  }

  // ---- the fused append's cache write (after every cache load of this workgroup) ---------------
  // Workgroup h writes its own slice [h*D/NSPLIT, (h+1)*D/NSPLIT) of the new K row and V^T
  // column. The other workgroup of the pair may still read that K row; it substitutes the
  // staged row for it, so what it reads does not matter.
  if (has_new) {
    constexpr int DS = D / NSPLIT;
    uint16_t* ck = reinterpret_cast<uint16_t*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D;
    uint16_t* cv = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
    for (int d = h * DS + tid; d < (h + 1) * DS; d += blockDim.x) {
      ck[kt_index(kr.new_slot, d, D)] = L.nk[d];
      cv[vt_index(kr.new_slot, d, D)] = L.nv[d];
    }
  }
  // lane (grp, col < R) holds O^T[d = 16*(dblock0 + ii) + 4*grp + j][head col]
  if (col < R) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)pair * R + col) * D;
#pragma unroll
    for (int ii = 0; ii < S::DPW; ++ii) {
      const uint32_t w0 = f32_to_bf16_bits(oacc[ii][0]) | (f32_to_bf16_bits(oacc[ii][1]) << 16);
      const uint32_t w1 = f32_to_bf16_bits(oacc[ii][2]) | (f32_to_bf16_bits(oacc[ii][3]) << 16);
      *reinterpret_cast<uint2*>(orow + 16 * (dblock0 + ii) + 4 * grp) = make_uint2(w0, w1);
    }
  }
}
