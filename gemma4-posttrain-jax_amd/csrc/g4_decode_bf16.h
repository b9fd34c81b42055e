// bf16 MFMA decode-attention kernels; included by g4_decode.hip inside namespace g4::{anon}.
//
// Lane roles for v_mfma_f32_16x16x32_bf16 (wave64): col = lane & 15, grp = lane >> 4.
//   QK  (S^T = K Q^T): A = 16 key rows x 32 d, B = 32 d x 16 query heads (R real, rest zero).
//       Block bb (0/1) of a 32-slot chunk puts slot c0 + 8*(m>>2) + 4*bb + (m&3) in A row m, so
//       the accumulator of lane (grp, col) holds head col's scores for slots c0 + 8*grp + e,
//       e = 4*bb + j — the B-operand layout of the value product below.
//   PV  (O^T = V^T P^T): A = 16 d rows x 32 slots of the transposed value cache (one 16-byte
//       buffer load per lane), B = probabilities of 32 slots x 16 heads, accumulators O^T[d, head].
//
// Memory-op order matters on gfx9: loads and stores share one in-order counter (vmcnt), so a
// wait for any load also waits for everything issued before it. The kernels therefore issue
// the small loads they need first (q and the appended token's K/V row, staged in LDS), then the
// cache loads, and write the appended row back to the cache last.

constexpr int NW = kDecodeWaves;

// LDS carve-up: scores f32 [R][t_alloc] | wave max [NW][16] | wave sum [NW][16] |
// q bf16 [R][D] | new K row, new V row bf16 [2][D] | probabilities bf16 [R][t_alloc].
// The O partials [NW][R][D] f32 alias from 0 once every wave is past its value pass.
struct DecodeLds {
  float* sc;
  float* wmax;
  float* wsum;
  uint16_t* qs;
  uint16_t* nk;
  uint16_t* nv;
  uint16_t* pl;
  float* red;
};

template <int D>
__device__ __forceinline__ DecodeLds carve(float* smem, int R, int t_alloc) {
  DecodeLds l;
  l.sc = smem;
  l.wmax = smem + R * t_alloc;
  l.wsum = l.wmax + NW * 16;
  l.qs = reinterpret_cast<uint16_t*>(l.wsum + NW * 16);
  l.nk = l.qs + R * D;
  l.nv = l.nk + D;
  l.pl = l.nv + D;
  l.red = smem;
  return l;
}

// q [R][D] and the appended token's K/V rows into LDS (the first global loads of the kernel).
template <int D>
__device__ __forceinline__ void stage_small(const G4DecodeArgs& a, int pair, const KeyRange& kr, const DecodeLds& L,
                                            int R) {
  const uint16_t* qh = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)pair * R * D;
  for (int i = threadIdx.x; i < R * D / 8; i += blockDim.x) reinterpret_cast<u32x4*>(L.qs)[i] = load16(qh + 8 * i);
  if (kr.new_slot >= 0) {
    const uint16_t* nk = reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D;
    const uint16_t* nv = reinterpret_cast<const uint16_t*>(a.new_v) + (int64_t)pair * D;
    for (int i = threadIdx.x; i < D / 8; i += blockDim.x) {
      reinterpret_cast<u32x4*>(L.nk)[i] = load16(nk + 8 * i);
      reinterpret_cast<u32x4*>(L.nv)[i] = load16(nv + 8 * i);
    }
  }
}

// The fused append's cache write (from LDS), issued after the kernel's last cache load. No
// other workgroup of this launch touches this (b, head), and the attention passes used the
// staged row, so the store only has to land before the next launch (stream order).
template <int D>
__device__ __forceinline__ void store_appended(const G4DecodeArgs& a, int pair, const KeyRange& kr,
                                               const DecodeLds& L) {
  if (kr.new_slot < 0) return;
  uint16_t* ck = reinterpret_cast<uint16_t*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D;
  uint16_t* cv = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    ck[kt_index(kr.new_slot, d, D)] = L.nk[d];
    cv[vt_index(kr.new_slot, d, D)] = L.nv[d];
  }
}

template <int D>
__device__ __forceinline__ bf16x8 q_operand(const uint16_t* qs, int R, int col, int grp, int s) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (col < R) v = *reinterpret_cast<const u32x4*>(qs + col * D + 32 * s + 8 * grp);
  return as_bf16x8(v);
}

// NT: non-temporal loads (no other workgroup reads these key rows).
template <int D, bool NT = false>
__device__ __forceinline__ void load_k_chunk(u32x4 (&kv)[2][D / 32], __amdgpu_buffer_rsrc_t rk, int c0, int col,
                                             int grp) {
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    // block (chunk, s, bb) of the key layout: lane (grp, col) reads 16 bytes at col * 64 + grp * 16
    const uint32_t voff = (uint32_t)((((c0 >> 5) * (D >> 5)) * 2 + bb) * 1024 + col * 64 + grp * 16);
#pragma unroll
    for (int s = 0; s < D / 32; ++s) kv[bb][s] = NT ? buffer_load16_nt(rk, voff + 2048u * s, 0u) : buffer_load16(rk, voff + 2048u * s, 0u);
  }
}

// Rows of the slot this launch appends come from the staged new K row.
template <int D>
__device__ __forceinline__ void patch_k(u32x4 (&kv)[2][D / 32], const uint16_t* nk, int64_t new_slot, int c0,
                                        int col, int grp) {
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const int kslot = c0 + 8 * (col >> 2) + 4 * bb + (col & 3);
    if (kslot == new_slot) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) kv[bb][s] = *reinterpret_cast<const u32x4*>(nk + 32 * s + 8 * grp);
    }
  }
}

// Scores of one chunk: MFMA, bf16 rounding, masking; stored to sc[col][slot]; running max.
template <int D>
__device__ __forceinline__ void score_chunk(const u32x4 (&kv)[2][D / 32], const uint16_t* qs, uint64_t vbits,
                                            float* sc, int t_alloc, int c0, int R, int col, int grp, float& mx) {
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) acc = mfma16x16x32(as_bf16x8(kv[bb][s]), q_operand<D>(qs, R, col, grp, s), acc);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = 8 * grp + 4 * bb + j;
      const float s = ((vbits >> kk) & 1ull) ? round_bf16(acc[j]) : kBf16Min;
      if (col < R) sc[col * t_alloc + c0 + kk] = s;
      mx = fmaxf(mx, s);
    }
  }
}

__device__ __forceinline__ uint64_t chunk_validity(const G4DecodeArgs& a, int b, const KeyRange& kr, int c0,
                                                   int lane) {
  return __ballot(key_valid(a, b, kr, c0 + (lane & 31)));
}

// key_valid without branches around the key_mask load (a clamped, always in-bounds byte read),
// so several chunks' validity loads can be in flight together.
__device__ __forceinline__ bool slot_valid_flat(const G4DecodeArgs& a, int b, const KeyRange& kr, int slot,
                                                uint8_t& maskbyte) {
  int64_t pos = slot;
  bool ok = slot < kr.n_keys;
  if (a.kind == G4_CACHE_RING) {
    pos = ring_slot_position(kr.q, slot, a.capacity);
    ok = ok && pos >= 0 && pos > kr.q - a.window;
  }
  ok = ok && pos <= kr.q && pos < a.key_mask_stride;
  const int64_t clamped = pos < 0 ? 0 : (pos >= a.key_mask_stride ? a.key_mask_stride - 1 : pos);
  maskbyte = a.key_mask[(int64_t)b * a.key_mask_stride + clamped];
  return ok;
}

template <int D>
__device__ __forceinline__ void load_v_chunk(u32x4 (&vv)[D / 16], __amdgpu_buffer_rsrc_t rv, int kb, int col) {
  const uint32_t voff = vt_operand_bytes(kb >> 3, col, D);
#pragma unroll
  for (int i = 0; i < D / 16; ++i) vv[i] = buffer_load16(rv, voff, 256u * i);  // value dims 16 i + col
}

// Replace the appended slot's value (if it falls in this lane's 8 slots) by the staged new V.
template <int D>
__device__ __forceinline__ void patch_v(u32x4 (&vv)[D / 16], const uint16_t* nv, int64_t new_slot, int kb, int col) {
  const int64_t off = new_slot - kb;
  if (off >= 0 && off < 8) {
    const int wsel = (int)(off >> 1);
    const bool hi = off & 1;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      const uint32_t nvb = nv[16 * i + col];
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // static indices only: no scratch copy of the vector
        const uint32_t word = vv[i][q];
        const uint32_t patched = hi ? ((word & 0x0000ffffu) | (nvb << 16)) : ((word & 0xffff0000u) | nvb);
        vv[i][q] = q == wsel ? patched : word;
      }
    }
  }
}

struct Softmax {
  float m, l;       // this lane's head (col < R)
  bool all_masked;  // no valid slot in the row: uniform 1/capacity over all slots
};

// Row max and sum over every scanned slot (two LDS rounds across the waves).
__device__ __forceinline__ Softmax softmax_stats(float mx, const float* sc, float* wmax, float* wsum, int t_alloc,
                                                 int n_chunks, int R, int w, int col, int grp) {
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (grp == 0) wmax[w * 16 + col] = mx;
  __syncthreads();
  Softmax sm;
  sm.m = kBf16Min;
  bool masked = true;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) {
    sm.m = fmaxf(sm.m, wmax[ww * 16 + col]);
    masked = masked && wmax[ww * 16] == kBf16Min;
  }
  sm.all_masked = masked;
  float l = 0.f;
  if (col < R) {
    for (int c = w; c < n_chunks; c += NW) {
      const float* sp = sc + col * t_alloc + (c << 5) + 8 * grp;
#pragma unroll
      for (int e = 0; e < 8; ++e) l += expf(sp[e] - sm.m);
    }
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (grp == 0) wsum[w * 16 + col] = l;
  __syncthreads();
  sm.l = 0.f;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) sm.l += wsum[ww * 16 + col];
  return sm;
}

// All threads: exact probabilities bf16(exp(s - m) / l) of slots [0, n_slots) into pl[R][t_alloc]
// (the m, l and summation order of softmax_stats), so the value pass reads one 16-byte LDS word
// per MFMA instead of holding exp/divide temporaries next to its V registers.
__device__ __forceinline__ void write_probs(const DecodeLds& L, int t_alloc, int n_slots, int R, bool all_masked,
                                            float p_uniform, int capacity) {
  for (int idx = threadIdx.x; idx < R * t_alloc; idx += blockDim.x) {
    const int r = idx / t_alloc, k = idx - r * t_alloc;
    if (k >= n_slots) continue;
    float p;
    if (all_masked) {
      p = k < capacity ? p_uniform : 0.f;
    } else {
      float m = kBf16Min, l = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) m = fmaxf(m, L.wmax[ww * 16 + r]);
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) l += L.wsum[ww * 16 + r];
      p = round_bf16(expf(L.sc[idx] - m) / l);
    }
    L.pl[idx] = (uint16_t)f32_to_bf16_bits(p);
  }
}

__device__ __forceinline__ bf16x8 prob_operand(const uint16_t* pl, int t_alloc, int kb, int R, int col) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (col < R) v = *reinterpret_cast<const u32x4*>(pl + col * t_alloc + kb);
  return as_bf16x8(v);
}

template <int D>
__device__ __forceinline__ void pv_chunk(const u32x4 (&vv)[D / 16], bf16x8 pop, floatx4 (&oacc)[D / 16]) {
#pragma unroll
  for (int i = 0; i < D / 16; ++i) oacc[i] = mfma16x16x32(as_bf16x8(vv[i]), pop, oacc[i]);
}

// Sum the waves' O^T partials in a fixed order and store bf16 [R][D].
template <int D>
__device__ __forceinline__ void reduce_store(const floatx4 (&oacc)[D / 16], float* red, uint16_t* out, int R, int w,
                                             int col, int grp) {
  __syncthreads();  // every wave is done with the LDS the partials overwrite
  if (col < R) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(w * R + col) * D + 16 * i + 4 * grp + j] = oacc[i][j];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * D; idx += blockDim.x) {
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) o += red[ww * R * D + idx];
    out[idx] = (uint16_t)f32_to_bf16_bits(o);
  }
}

// General kernel: any number of 32-slot chunks (each wave loops over chunks w, w+NW, ...),
// slots [0, t_alloc) of the probabilities live in LDS.
template <int D>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_bf16_kernel(G4DecodeArgs a, int t_alloc) {
  constexpr int DB = D / 16;
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
  stage_small<D>(a, pair, kr, L, R);
  __syncthreads();

  const int n_chunks = (kr.n_keys + 31) >> 5;
  float mx = kBf16Min;
  for (int c = w; c < n_chunks; c += NW) {
    const int c0 = c << 5;
    u32x4 kv[2][D / 32];
    load_k_chunk<D>(kv, rk, c0, col, grp);
    patch_k<D>(kv, L.nk, kr.new_slot, c0, col, grp);
    score_chunk<D>(kv, L.qs, chunk_validity(a, b, kr, c0, lane), L.sc, t_alloc, c0, R, col, grp, mx);
  }
  const Softmax sm = softmax_stats(mx, L.sc, L.wmax, L.wsum, t_alloc, n_chunks, R, w, col, grp);
  const int n_chunks2 = ((sm.all_masked ? a.capacity : kr.n_keys) + 31) >> 5;
  write_probs(L, t_alloc, n_chunks2 << 5, R, sm.all_masked, round_bf16(1.0f / (float)a.capacity), a.capacity);
  __syncthreads();

  floatx4 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c = w; c < n_chunks2; c += NW) {
    const int kb = (c << 5) + 8 * grp;
    u32x4 vv[DB];
    load_v_chunk<D>(vv, rv, kb, col);
    patch_v<D>(vv, L.nv, kr.new_slot, kb, col);
    pv_chunk<D>(vv, prob_operand(L.pl, t_alloc, kb, R, col), oacc);
  }
  store_appended<D>(a, pair, kr, L);  // before reduce_store: its partials overwrite the staged rows
  reduce_store<D>(oacc, L.red, reinterpret_cast<uint16_t*>(a.out) + (int64_t)pair * R * D, R, w, col, grp);
}
