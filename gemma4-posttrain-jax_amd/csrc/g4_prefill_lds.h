// bf16 prefill attention with the key / value chunks staged through LDS (head dims 128, 256);
// included by g4_prefill.hip after prefill_bf16_kernel.
//
// A workgroup of NW waves owns NW * NB * 16/R consecutive query positions of one (b, kv head);
// each wave owns NB column blocks of 16 query rows (16/R positions x R heads each), so every K and
// V^T operand tile it reads from LDS feeds NB MFMAs. The key range is walked in 32-key chunks:
// every chunk's K and V^T are DMA'd into LDS once per workgroup (buffer_load ... lds, each wave
// issuing an equal share, into rings of 4 slots) as lane-ordered MFMA operand tiles, and all waves
// read them from there. The key-mask bytes of the row are staged in LDS once, so a chunk's validity
// is one LDS byte per lane and a ballot.
//
// Same two passes as prefill_bf16_kernel (the reference rounds probabilities after the full-row
// softmax): pass 1 streams K for each row's max and sum, pass 2 streams K and V and forms the bf16
// probabilities of the full-row softmax for the value product, evaluated as __expf(s - m) * (1/l):
// the hardware exp and the row's reciprocal instead of expf and a division per score, a few f32
// ulps from exp(s - m) / l, so a probability at a bf16 rounding boundary may round one bf16 step
// the other way. Workgroups are launched heaviest (latest positions, longest causal key range)
// first.
//
// What bounds it is the issue rate of each SIMD's two waves, VALU work included, more than the
// MFMAs, so the schedule is built around three things:
//  - a wave-uniform fast path: a chunk whose 32 keys every row of the wave may see (key mask,
//    causal limit, window) skips the per-key selects, and its scores are rounded two per
//    conversion instruction;
//  - operand tiles read from LDS through a rolling window: tile t + W is requested right after the
//    MFMAs of tile t, so the LDS latency hides behind the MFMAs in flight;
//  - in pass 2 the two waves sharing a SIMD (w, w + NW/2) are half a step apart. One runs the
//    MFMA phase (the values of chunk c-1, then the QK of chunk c) while the other runs the VALU
//    phase (the probabilities of a chunk), at raised priority while in the MFMA phase.

constexpr int kPfMaxSeq = 32768;  // key-mask bytes staged in LDS

template <int D, int NW>
struct PfShape {
  static constexpr int KT = 2 * (D / 32);  // K operand tiles per chunk: (bb, s)
  static constexpr int VT = D / 16;        // V^T operand tiles per chunk: d-blocks
  static constexpr int KT_W = KT / NW;     // DMA'd by each wave
  static constexpr int VT_W = VT / NW;
  static_assert(KT % NW == 0 && VT % NW == 0, "tiles split evenly over the waves");
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The 8 scores of one column block (both 16-key halves), each rounded to bf16, two values per
// conversion instruction; element e is key 8 * grp + e of the chunk.
__device__ __forceinline__ void pf_round8(const floatx4 (&acc)[2], float (&sc)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = pack_bf16x2(acc[j >> 1][2 * (j & 1)], acc[j >> 1][2 * (j & 1) + 1]);
    sc[2 * j] = __uint_as_float(w << 16);
    sc[2 * j + 1] = __uint_as_float(w & 0xffff0000u);
  }
}

// S^T of one chunk for the wave's NB column blocks: K operand tiles (KT = 2 halves x KS d-slices,
// 1 KiB each from LDS address kbase) against the q operands in registers, a rolling window of WIN
// tiles in flight (each read waited for right before its MFMAs; the chunk's DMA is covered by the
// caller's vmcnt wait + barrier).
template <int KT, int KS, int NB, int WIN>
__device__ __forceinline__ void pf_qk(uint32_t kbase, const bf16x8 (&qop)[NB][KS], floatx4 (&acc)[NB][2], int lane) {
  static_assert(WIN >= 1 && WIN <= 8 && WIN <= KT, "window of LDS reads (lgkm_wait counts up to 7)");
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) acc[cb][0] = acc[cb][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  u32x4 kv[WIN];
#pragma unroll
  for (int j = 0; j < WIN; ++j) kv[j] = lds_read16(kbase + 1024u * j + 16u * lane);
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int bb = t / KS, s = t - bb * KS;
    const int later = KT - 1 - t < WIN - 1 ? KT - 1 - t : WIN - 1;  // reads issued after tile t's
    lgkm_wait(later, kv[t % WIN]);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) acc[cb][bb] = mfma16x16x32(as_bf16x8(kv[t % WIN]), qop[cb][s], acc[cb][bb]);
    if (t + WIN < KT) kv[t % WIN] = lds_read16(kbase + 1024u * (t + WIN) + 16u * lane);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// O^T += V^T P^T over one chunk: VT value operand tiles (one per 16-dim block, 1 KiB each from LDS
// address vbase) against the wave's probabilities, a rolling window of WIN tiles in flight.
template <int VT, int NB, int WIN>
__device__ __forceinline__ void pf_pv(uint32_t vbase, const bf16x8 (&pop)[NB], floatx4 (&oacc)[NB][VT], int lane) {
  static_assert(WIN >= 1 && WIN <= 8 && WIN <= VT, "window of LDS reads (lgkm_wait counts up to 7)");
  __builtin_amdgcn_sched_barrier(0);
  u32x4 vv[WIN];
#pragma unroll
  for (int i = 0; i < WIN; ++i) vv[i] = lds_read16(vbase + 1024u * i + 16u * lane);
#pragma unroll
  for (int i = 0; i < VT; ++i) {
    const int later = VT - 1 - i < WIN - 1 ? VT - 1 - i : WIN - 1;
    lgkm_wait(later, vv[i % WIN]);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) oacc[cb][i] = mfma16x16x32(as_bf16x8(vv[i % WIN]), pop[cb], oacc[cb][i]);
    if (i + WIN < VT) vv[i % WIN] = lds_read16(vbase + 1024u * (i + WIN) + 16u * lane);
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int D, int NB, int NW>
__global__ __launch_bounds__(NW * 64) void prefill_bf16_lds_kernel(G4PrefillArgs a) {
  using S_ = PfShape<D, NW>;
  constexpr int KS = D / 32;
  // the ring slots as separate arrays, so the compiler's wait before reading one does not include
  // the DMA still in flight into the others
  __shared__ __attribute__((aligned(1024))) unsigned char kb0[S_::KT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char vb0[S_::VT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char kb1[S_::KT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char vb1[S_::VT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char kb2[S_::KT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char vb2[S_::VT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char kb3[S_::KT][1024];
  __shared__ __attribute__((aligned(1024))) unsigned char vb3[S_::VT][1024];
  extern __shared__ float smem[];
  uint8_t* km_lds = reinterpret_cast<uint8_t*>(smem);  // key_mask[b, 0:S]

  const int R = a.group;
  const int ppc = 16 / R;              // positions per 16-row column block
  const int ppw = NB * ppc;            // positions per wave
  const int ppb = NW * ppw;            // positions per workgroup
  const int S = a.seq, H = a.kv_heads;
  const int nblk = (S + ppb - 1) / ppb;
  // One-dimensional grid. Causal rows (no window, or one that spans the sequence): a block's cost
  // grows with its position, so workgroup i takes block nblk - 1 - i / (B H) of pair i % (B H): the
  // latest blocks of every pair are dispatched before anyone's shorter ones (config 4's global layer:
  // 1.10 -> 0.99 ms against pair-major order). Windowed rows cost the same from block to block;
  // pair-major order (workgroup i: block nblk - 1 - i % nblk of pair i / nblk) keeps the workgroups in
  // flight on different key offsets, which measured faster there (sliding layer 0.36 against
  // 0.49 ms block-major). There, with a multiple of 8 pairs, consecutive blocks of a pair go to one
  // XCD (workgroups are dealt to the 8 XCDs round robin, i mod 8), so the overlapping key windows
  // of neighbouring blocks meet in one L2 (0.290-0.294 -> 0.278-0.283 ms); block-major order already
  // keeps a pair on one XCD.
  const int npairs = a.batch * H;
  const bool blk_major = a.window <= 0 || a.window >= S;
  int blk, pair;
  if (blk_major) {
    blk = nblk - 1 - (int)(blockIdx.x / (unsigned)npairs);
    pair = (int)(blockIdx.x % (unsigned)npairs);
  } else if (npairs % 8 == 0) {
    const int i = (int)blockIdx.x, j = i >> 3;
    blk = nblk - 1 - j % nblk;
    pair = (j / nblk) * 8 + (i & 7);
  } else {
    blk = nblk - 1 - (int)(blockIdx.x % (unsigned)nblk);
    pair = (int)(blockIdx.x / (unsigned)nblk);
  }
  const int b = pair / H, h = pair - b * H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int p0 = blk * ppb;                       // first position of the workgroup
  const int r = col - (col / R) * R;
  int my_pos[NB];                                 // this lane's query row (column col) of each block
  bool row_ok[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    my_pos[cb] = p0 + w * ppw + cb * ppc + col / R;
    row_ok[cb] = my_pos[cb] < S;
  }
  const int64_t bh = (int64_t)b * H + h;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(reinterpret_cast<const uint16_t*>(a.k) + bh * a.k_stride * D,
                                              (uint32_t)a.k_stride * D * 2u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(reinterpret_cast<const uint16_t*>(a.vt) + bh * D * a.k_stride,
                                              (uint32_t)a.k_stride * D * 2u);

  // q operands (registers) and the row's key-mask bytes (LDS)
  bf16x8 qop[NB][KS];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const uint16_t* qrow =
        reinterpret_cast<const uint16_t*>(a.q) + ((((int64_t)b * S + my_pos[cb]) * H + h) * R + r) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row_ok[cb]) v = load16(qrow + 32 * s + 8 * grp);
      qop[cb][s] = as_bf16x8(v);
    }
  }
  const uint8_t* km = a.key_mask + (int64_t)b * a.key_mask_stride;
  for (int i = tid; i < S; i += blockDim.x) km_lds[i] = km[i];

  const int pos_last = min(p0 + ppb - 1, S - 1);
  const int kmin = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
  const int c_begin = kmin >> 5, c_end = pos_last >> 5;

  // This wave's share of a chunk's K / V^T operand tiles into LDS. Both layouts put chunk c at byte
  // 64 * D * c, so a tile's lane offset does not depend on the chunk, which rides in soffset (every
  // chunk issued lies inside the cache rows: c <= (S - 1) / 32 and S <= k_stride).
  auto issue_k = [&](int c, unsigned char (&kt)[S_::KT][1024]) {
    const uint32_t cofs = (uint32_t)c * (uint32_t)(64 * D);
#pragma unroll
    for (int i = 0; i < S_::KT_W; ++i) {
      const int t = w * S_::KT_W + i, bb = t / KS, s = t - bb * KS;
      const uint32_t ko = (uint32_t)kt_index(8 * (col >> 2) + 4 * bb + (col & 3), 32 * s + 8 * grp, D) * 2u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)&kt[t][0], 16, ko, cofs, 0, 0);
    }
  };
  auto issue_v = [&](int c, unsigned char (&vt)[S_::VT][1024]) {
    const uint32_t cofs = (uint32_t)c * (uint32_t)(64 * D);
#pragma unroll
    for (int i = 0; i < S_::VT_W; ++i) {
      const int t = w * S_::VT_W + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)&vt[t][0], 16,
                                               vt_operand_bytes(grp, 16 * t + col, D), cofs, 0, 0);
    }
  };
  // key-mask ballot of the chunk's 32 keys (lanes l and l + 32 both hold key 32 c + l % 32)
  auto chunk_ballot = [&](int c) -> uint64_t {
    const int key = (c << 5) + (lane & 31);
    return __ballot(key < S && km_lds[key < S ? key : 0] != 0);
  };
  // Wave-uniform: every row of this wave sees all 32 keys of chunk c (key mask, causal limit,
  // window, rows inside the sequence).
  const int wpos_min = p0 + w * ppw;
  const int wpos_max = wpos_min + (NB - 1) * ppc + 15 / R;
  auto chunk_full = [&](int c, uint64_t mb) -> bool {
    const int k0 = c << 5;
    return (uint32_t)mb == 0xffffffffu && k0 + 31 <= wpos_min && wpos_max < S &&
           (a.window <= 0 || k0 >= wpos_max - a.window + 1);
  };
  // this lane's key bits of the chunk (bit e <-> key 32 c + 8 grp + e) for block cb's row: the key
  // mask, causal, and the window
  auto valid_bits = [&](int c, uint64_t mb, int cb) -> uint32_t {
    uint32_t bits = (uint32_t)(mb >> (8 * grp)) & 0xffu;
    const int lo = (c << 5) + 8 * grp;
    const int hi_ok = my_pos[cb] - lo;  // keys lo + e valid for e <= hi_ok
    bits &= hi_ok >= 7 ? 0xffu : (hi_ok < 0 ? 0u : (0xffu >> (7 - hi_ok)));
    if (a.window > 0) {
      const int lo_ok = my_pos[cb] - a.window + 1 - lo;  // need e >= lo_ok
      bits &= lo_ok <= 0 ? 0xffu : (lo_ok > 7 ? 0u : (0xffu << lo_ok) & 0xffu);
    }
    return row_ok[cb] ? bits : 0u;
  };

  // ---- pass 1: row max and sum --------------------------------------------------------------------
  float m[NB], l[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    m[cb] = kBf16Min;
    l[cb] = 0.f;
  }
  // one rescale per chunk: l <- l * exp(m - m') + sum exp(s - m') with m' = max(m, chunk max)
  // (masked keys score the fill value, whose exp vanishes against any real maximum)
  auto stats = [&](int c, unsigned char (&kt)[S_::KT][1024]) {
    floatx4 acc[NB][2];
    pf_qk<S_::KT, KS, NB, 8>(lds_addr(&kt[0][0]), qop, acc, lane);  // pass 1 holds no value accumulators
    const uint64_t mb = chunk_ballot(c);
    if (chunk_full(c, mb)) {
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        float sc[8], mx = kBf16Min;
        pf_round8(acc[cb], sc);
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, sc[e]);
        const float mn = fmaxf(m[cb], mx);
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += __expf(sc[e] - mn);
        l[cb] = l[cb] * __expf(m[cb] - mn) + sum;
        m[cb] = mn;
      }
      return;
    }
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const uint32_t bits = valid_bits(c, mb, cb);
      float sc[8], mx = kBf16Min;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sc[e] = ((bits >> e) & 1u) ? round_bf16(acc[cb][e >> 2][e & 3]) : kBf16Min;
        mx = fmaxf(mx, sc[e]);
      }
      const float mn = fmaxf(m[cb], mx);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += __expf(sc[e] - mn);
      l[cb] = l[cb] * __expf(m[cb] - mn) + sum;
      m[cb] = mn;
    }
  };
  // One pipeline step: wait for this wave's DMA of chunk c (chunks c+1, c+2 may stay in flight),
  // barrier (every wave's share of chunk c has landed, and every wave is done with chunk c-1, whose
  // slot the DMA of chunk c+3 reuses), queue chunk c+3, compute chunk c.
  auto wait_chunk = [&](int c, int c_last) {
    constexpr int n = S_::KT_W;
    const int ahead = min(c_last - c, 2);  // chunks queued after c
    if (ahead >= 2) wait_vmcnt<2 * n>();
    else if (ahead == 1) wait_vmcnt<n>();
    else wait_vmcnt<0>();
    wg_barrier();
  };
  __syncthreads();  // key-mask bytes in LDS (no DMA in flight yet)
  issue_k(c_begin, kb0);
  if (c_begin + 1 <= c_end) issue_k(c_begin + 1, kb1);
  if (c_begin + 2 <= c_end) issue_k(c_begin + 2, kb2);
  // (guarded steps rather than early exits: the accumulators then merge at one point per step)
  for (int c = c_begin; c <= c_end; c += 4) {
    wait_chunk(c, c_end);
    if (c + 3 <= c_end) issue_k(c + 3, kb3);
    stats(c, kb0);
    if (c + 1 <= c_end) {
      wait_chunk(c + 1, c_end);
      if (c + 4 <= c_end) issue_k(c + 4, kb0);
      stats(c + 1, kb1);
    }
    if (c + 2 <= c_end) {
      wait_chunk(c + 2, c_end);
      if (c + 5 <= c_end) issue_k(c + 5, kb1);
      stats(c + 2, kb2);
    }
    if (c + 3 <= c_end) {
      wait_chunk(c + 3, c_end);
      if (c + 6 <= c_end) issue_k(c + 6, kb2);
      stats(c + 3, kb3);
    }
  }
  bool row_masked[NB], mine_masked = false;
  float rl[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
#pragma unroll
    for (int msk = 16; msk <= 32; msk <<= 1) {
      const float m2 = __shfl_xor(m[cb], msk, 64);
      const float l2 = __shfl_xor(l[cb], msk, 64);
      const float mm = fmaxf(m[cb], m2);
      l[cb] = l[cb] * __expf(m[cb] - mm) + l2 * __expf(m2 - mm);
      m[cb] = mm;
    }
    // A row with no valid key is the reference's softmax over S equal fills: 1/S on every key.
    row_masked[cb] = row_ok[cb] && m[cb] == kBf16Min;
    mine_masked = mine_masked || row_masked[cb];
    rl[cb] = 1.0f / l[cb];
  }
  const bool any_masked = __syncthreads_or(mine_masked);  // (also: every wave is done with pass 1's LDS)
  const float p_uniform = round_bf16(1.0f / (float)S);
  const int c2_begin = any_masked ? 0 : c_begin;
  const int c2_end = any_masked ? (S - 1) >> 5 : c_end;

  // ---- pass 2: exact probabilities and O^T = V^T P^T -------------------------------------------------
  floatx4 oacc[NB][S_::VT];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb)
#pragma unroll
    for (int i = 0; i < S_::VT; ++i) oacc[cb][i] = floatx4{0.f, 0.f, 0.f, 0.f};
  // exact bf16 probabilities of chunk c from its score accumulators (the B operand of O^T += V^T P^T)
  auto probs = [&](int c, const floatx4 (&acc)[NB][2], bf16x8 (&pop)[NB]) {
    const uint64_t mb = chunk_ballot(c);
    if (!any_masked && chunk_full(c, mb)) {
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        float sc[8], p[8];
        pf_round8(acc[cb], sc);
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = __expf(sc[e] - m[cb]) * rl[cb];
        pop[cb] = as_bf16x8(u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                  pack_bf16x2(p[6], p[7])});
      }
      return;
    }
    const int kb = (c << 5) + 8 * grp;
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const uint32_t bits = valid_bits(c, mb, cb);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (row_masked[cb]) p[e] = kb + e < S ? p_uniform : 0.f;
        else p[e] = ((bits >> e) & 1u) ? __expf(round_bf16(acc[cb][e >> 2][e & 3]) - m[cb]) * rl[cb] : 0.f;
      }
      pop[cb] = as_bf16x8(u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                pack_bf16x2(p[6], p[7])});
    }
  };
  // One barrier per chunk step. After the barrier of chunk c every wave runs two phases:
  // M(c) = the values of chunk c-1 (its V^T tiles x the probabilities formed earlier) and the QK of
  // chunk c (MFMA work), and P(c) = the probabilities of chunk c (VALU work). Waves 0..NW/2-1 run
  // M(c) then P(c); waves NW/2.. run P(c-1) then M(c). Chunk j sits in slot (j - c2_begin) % 4 of
  // both rings; K(c) and V(c-1) are read only in step c, and the barrier of chunk c queues K(c+3)
  // and V(c+2) into the slots of K(c-1) and V(c-2), which step c-1 finished reading.
  const bool lead = w < NW / 2;
  // this wave's DMAs of K(c) and V(c-1) have landed: queued after them are V(c) and, where they
  // exist, K(c+1), K(c+2) and V(c+1)
  auto wait_step = [&](int c, int c_last) {
    constexpr int nk = S_::KT_W, nv = S_::VT_W;
    if (c + 2 <= c_last) wait_vmcnt<2 * nk + 2 * nv>();
    else if (c + 1 <= c_last) wait_vmcnt<nk + 2 * nv>();
    else wait_vmcnt<nv>();
    wg_barrier();
  };
  floatx4 acc[NB][2];
  bf16x8 pop[NB];
  auto p2_step = [&](int c, unsigned char (&kcur)[S_::KT][1024], unsigned char (&vprev)[S_::VT][1024],
                     unsigned char (&knext)[S_::KT][1024], unsigned char (&vnext)[S_::VT][1024]) {
    wait_step(c, c2_end);
    if (c + 3 <= c2_end) issue_k(c + 3, knext);
    if (c + 2 <= c2_end) issue_v(c + 2, vnext);
    if (!lead && c > c2_begin) probs(c - 1, acc, pop);
    __builtin_amdgcn_s_setprio(1);
    if (c > c2_begin) pf_pv<S_::VT, NB, 4>(lds_addr(&vprev[0][0]), pop, oacc, lane);
    pf_qk<S_::KT, KS, NB, 4>(lds_addr(&kcur[0][0]), qop, acc, lane);
    __builtin_amdgcn_s_setprio(0);
    if (lead) probs(c, acc, pop);
  };
  // prologue, in the steady state's order: K(b), K(b+1), V(b), K(b+2), V(b+1) (b = c2_begin <= c2_end:
  // a row's own position is one of its keys)
  issue_k(c2_begin, kb0);
  if (c2_begin + 1 <= c2_end) issue_k(c2_begin + 1, kb1);
  issue_v(c2_begin, vb0);
  if (c2_begin + 2 <= c2_end) issue_k(c2_begin + 2, kb2);
  if (c2_begin + 1 <= c2_end) issue_v(c2_begin + 1, vb1);
  for (int c = c2_begin; c <= c2_end; c += 4) {  // guarded steps: the accumulators merge once per step
    p2_step(c, kb0, vb3, kb3, vb2);
    if (c + 1 <= c2_end) p2_step(c + 1, kb1, vb0, kb0, vb3);
    if (c + 2 <= c2_end) p2_step(c + 2, kb2, vb1, kb1, vb0);
    if (c + 3 <= c2_end) p2_step(c + 3, kb3, vb2, kb2, vb1);
  }
  // the last chunk's values: every wave's share of its V^T tiles has landed after this barrier
  wait_vmcnt<0>();
  wg_barrier();
  if (!lead) probs(c2_end, acc, pop);
  {
    const int slot = (c2_end - c2_begin) & 3;
    const uint32_t vlast = slot == 0   ? lds_addr(&vb0[0][0])
                           : slot == 1 ? lds_addr(&vb1[0][0])
                           : slot == 2 ? lds_addr(&vb2[0][0])
                                       : lds_addr(&vb3[0][0]);
    pf_pv<S_::VT, NB, 4>(vlast, pop, oacc, lane);
  }

#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    if (row_ok[cb]) {
      uint16_t* orow =
          reinterpret_cast<uint16_t*>(a.out) + ((((int64_t)b * S + my_pos[cb]) * H + h) * R + r) * D;
#pragma unroll
      for (int i = 0; i < S_::VT; ++i) {
        *reinterpret_cast<uint2*>(orow + 16 * i + 4 * grp) =
            make_uint2(pack_bf16x2(oacc[cb][i][0], oacc[cb][i][1]), pack_bf16x2(oacc[cb][i][2], oacc[cb][i][3]));
      }
    }
  }
}
