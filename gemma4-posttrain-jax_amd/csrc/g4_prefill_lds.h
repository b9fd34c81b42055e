// bf16 prefill attention with the key / value chunks staged through LDS (head dims 128, 256);
// included by g4_prefill.hip after prefill_bf16_kernel.
//
// A workgroup of NW waves owns NW * NB * 16/R consecutive query positions of one (b, kv head);
// each wave owns NB column blocks of 16 query rows (16/R positions x R heads each), so every K and
// V^T operand tile it reads from LDS feeds NB MFMAs. The key range is
// walked in 32-key chunks: every chunk's K and V^T are DMA'd into LDS once per workgroup
// (buffer_load ... lds through a ring of 4 buffers, three chunks in flight ahead of the one being
// computed, each wave issuing an equal share) as lane-ordered
// MFMA operand tiles, and all 8 waves read them from there — against 1 KiB of global loads per
// MFMA when each wave loads its own operands. The key-mask bytes of the row are staged in LDS
// once, so a chunk's validity bits are one LDS byte per lane and a ballot.
//
// Same two passes as prefill_bf16_kernel (the reference rounds probabilities after the full-row
// softmax): pass 1 streams K for each row's max and sum, pass 2 streams K and V and forms exact
// bf16 probabilities exp(s - m) * (1/l) for the value product. Workgroups are launched heaviest
// (latest positions, longest causal key range) first.

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

template <int D, int NB, int NW>
__global__ __launch_bounds__(NW * 64) void prefill_bf16_lds_kernel(G4PrefillArgs a) {
  using S_ = PfShape<D, NW>;
  constexpr int KS = D / 32;
  // four buffers as separate arrays, so the compiler's wait before reading one does not include
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
  const int b = blockIdx.z, h = blockIdx.y;
  const int nblk = (S + ppb - 1) / ppb;
  const int blk = nblk - 1 - (int)blockIdx.x;  // heaviest first
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

  // this wave's share of a chunk's operand tiles into LDS
  auto issue = [&](int c, unsigned char (&kt)[S_::KT][1024], unsigned char (&vt)[S_::VT][1024], bool with_v) {
    const int c0 = c << 5;
#pragma unroll
    for (int i = 0; i < S_::KT_W; ++i) {
      const int t = w * S_::KT_W + i, bb = t / KS, s = t - bb * KS;
      const int key = c0 + 8 * (col >> 2) + 4 * bb + (col & 3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)&kt[t][0], 16,
                                               (uint32_t)kt_index(key, 32 * s + 8 * grp, D) * 2u, 0, 0, 0);
    }
    if (with_v) {
#pragma unroll
      for (int i = 0; i < S_::VT_W; ++i) {
        const int t = w * S_::VT_W + i;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rv, (__attribute__((address_space(3))) void*)&vt[t][0], 16,
            vt_operand_bytes(4 * c + grp, 16 * t + col, D), 0, 0, 0);
      }
    }
  };
  // key-mask bits of the chunk's 32 keys (bit e <-> key c0 + 8*grp + e), shared by the blocks
  auto mask_bits = [&](int c) -> uint32_t {
    const int key = (c << 5) + (lane & 31);
    const uint64_t mb = __ballot(key < S && km_lds[key < S ? key : 0] != 0);
    return (uint32_t)(mb >> (8 * grp)) & 0xffu;
  };
  // ... restricted to the keys block cb's row may see: causal, and the window
  auto valid_bits = [&](int c, uint32_t bits, int cb) -> uint32_t {
    const int lo = (c << 5) + 8 * grp;
    const int hi_ok = my_pos[cb] - lo;  // keys lo + e valid for e <= hi_ok
    bits &= hi_ok >= 7 ? 0xffu : (hi_ok < 0 ? 0u : (0xffu >> (7 - hi_ok)));
    if (a.window > 0) {
      const int lo_ok = my_pos[cb] - a.window + 1 - lo;  // need e >= lo_ok
      bits &= lo_ok <= 0 ? 0xffu : (lo_ok > 7 ? 0u : (0xffu << lo_ok) & 0xffu);
    }
    return row_ok[cb] ? bits : 0u;
  };
  // scores of both 16-key halves (bb) for every block: each K tile is read once for NB MFMAs
  // (the scheduling barriers bound how many operand tiles are read ahead into registers)
  auto qk = [&](unsigned char (&kt)[S_::KT][1024], floatx4 (&acc)[NB][2]) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      floatx4 x[NB];
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) x[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
      // the K tiles are read by inline-assembly LDS reads, each waited for right before its MFMAs
      // (the DMA of this chunk is covered by wait_chunk's vmcnt + barrier)
      constexpr int KG = KS < 4 ? KS : 4;  // tiles read ahead (bounds the registers they hold)
#pragma unroll
      for (int s0 = 0; s0 < KS; s0 += KG) {
        u32x4 kv[KG];
#pragma unroll
        for (int j = 0; j < KG; ++j) kv[j] = lds_read16(lds_addr(&kt[bb * KS + s0 + j][16 * lane]));
#pragma unroll
        for (int j = 0; j < KG; ++j) {
          lgkm_wait(KG - 1 - j, kv[j]);
#pragma unroll
          for (int cb = 0; cb < NB; ++cb) x[cb] = mfma16x16x32(as_bf16x8(kv[j]), qop[cb][s0 + j], x[cb]);
        }
      }
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) acc[cb][bb] = x[cb];
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- pass 1: row max and sum --------------------------------------------------------------------
  float m[NB], l[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    m[cb] = kBf16Min;
    l[cb] = 0.f;
  }
  auto stats = [&](int c, unsigned char (&kt)[S_::KT][1024]) {
    floatx4 acc[NB][2];
    qk(kt, acc);
    const uint32_t mbits = mask_bits(c);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      // one rescale per chunk: l <- l * exp(m - m') + sum exp(s - m') with m' = max(m, chunk max)
      // (masked keys score the fill value, whose exp vanishes against any real maximum)
      const uint32_t bits = valid_bits(c, mbits, cb);
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
  // buffer the DMA of chunk c+3 reuses), queue chunk c+3, compute chunk c.
  auto wait_chunk = [&](int c, int c_last, bool with_v) {
    const int ahead = min(c_last - c, 2);  // chunks queued after c
    if (with_v) {
      constexpr int n = S_::KT_W + S_::VT_W;
      if (ahead >= 2) wait_vmcnt<2 * n>();
      else if (ahead == 1) wait_vmcnt<n>();
      else wait_vmcnt<0>();
    } else {
      constexpr int n = S_::KT_W;
      if (ahead >= 2) wait_vmcnt<2 * n>();
      else if (ahead == 1) wait_vmcnt<n>();
      else wait_vmcnt<0>();
    }
    wg_barrier();
  };
  __syncthreads();  // key-mask bytes in LDS (no DMA in flight yet)
  issue(c_begin, kb0, vb0, false);
  if (c_begin + 1 <= c_end) issue(c_begin + 1, kb1, vb1, false);
  if (c_begin + 2 <= c_end) issue(c_begin + 2, kb2, vb2, false);
  // (guarded steps rather than early exits: the accumulators then merge at one point per step)
  for (int c = c_begin; c <= c_end; c += 4) {
    wait_chunk(c, c_end, false);
    if (c + 3 <= c_end) issue(c + 3, kb3, vb3, false);
    stats(c, kb0);
    if (c + 1 <= c_end) {
      wait_chunk(c + 1, c_end, false);
      if (c + 4 <= c_end) issue(c + 4, kb0, vb0, false);
      stats(c + 1, kb1);
    }
    if (c + 2 <= c_end) {
      wait_chunk(c + 2, c_end, false);
      if (c + 5 <= c_end) issue(c + 5, kb1, vb1, false);
      stats(c + 2, kb2);
    }
    if (c + 3 <= c_end) {
      wait_chunk(c + 3, c_end, false);
      if (c + 6 <= c_end) issue(c + 6, kb2, vb2, false);
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
  auto values = [&](int c, unsigned char (&kt)[S_::KT][1024], unsigned char (&vt)[S_::VT][1024]) {
    floatx4 acc[NB][2];
    qk(kt, acc);
    const uint32_t mbits = mask_bits(c);
    const int kb = (c << 5) + 8 * grp;
    bf16x8 pop[NB];
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const uint32_t bits = valid_bits(c, mbits, cb);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (row_masked[cb]) p[e] = kb + e < S ? p_uniform : 0.f;
        else p[e] = ((bits >> e) & 1u) ? __expf(round_bf16(acc[cb][e >> 2][e & 3]) - m[cb]) * rl[cb] : 0.f;
      }
      pop[cb] = as_bf16x8(u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                pack_bf16x2(p[6], p[7])});
    }
    constexpr int GRP = 8 / NB;  // V tiles read ahead per scheduling group
#pragma unroll
    for (int i0 = 0; i0 < S_::VT; i0 += GRP) {
      __builtin_amdgcn_sched_barrier(0);
      u32x4 vv[GRP];
#pragma unroll
      for (int i = i0; i < i0 + GRP && i < S_::VT; ++i) vv[i - i0] = lds_read16(lds_addr(&vt[i][16 * lane]));
#pragma unroll
      for (int i = i0; i < i0 + GRP && i < S_::VT; ++i) {
        lgkm_wait((i0 + GRP < S_::VT ? i0 + GRP : S_::VT) - 1 - i, vv[i - i0]);
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) oacc[cb][i] = mfma16x16x32(as_bf16x8(vv[i - i0]), pop[cb], oacc[cb][i]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  issue(c2_begin, kb0, vb0, true);
  if (c2_begin + 1 <= c2_end) issue(c2_begin + 1, kb1, vb1, true);
  if (c2_begin + 2 <= c2_end) issue(c2_begin + 2, kb2, vb2, true);
  for (int c = c2_begin; c <= c2_end; c += 4) {
    wait_chunk(c, c2_end, true);
    if (c + 3 <= c2_end) issue(c + 3, kb3, vb3, true);
    values(c, kb0, vb0);
    if (c + 1 <= c2_end) {
      wait_chunk(c + 1, c2_end, true);
      if (c + 4 <= c2_end) issue(c + 4, kb0, vb0, true);
      values(c + 1, kb1, vb1);
    }
    if (c + 2 <= c2_end) {
      wait_chunk(c + 2, c2_end, true);
      if (c + 5 <= c2_end) issue(c + 5, kb1, vb1, true);
      values(c + 2, kb2, vb2);
    }
    if (c + 3 <= c2_end) {
      wait_chunk(c + 3, c2_end, true);
      if (c + 6 <= c2_end) issue(c + 6, kb2, vb2, true);
      values(c + 3, kb3, vb3);
    }
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
