// bf16 decode attention in two stream-ordered launches, for rows of at most 1024 slots over many
// (b, kv head) pairs (the E2B rollout batch: the 512-slot sliding-window ring and the global
// layers' linear cache); included by g4_decode.hip after g4_decode_splitk.h.
//
// The one-launch kernels keep a pair's whole row on one CU: K streams in, the row is scored, the
// softmax runs behind barriers and the value pass follows, so every CU ends each pair with a
// compute tail during which it has no loads in flight. Here each launch is a plain stream of
// small independent workgroups, so one workgroup's tail overlaps the next one's loads:
//   scores  one wave per 32-slot chunk: K into registers, MFMA against the q operand (read from
//           LDS from head dim 256), bf16-rounded masked scores into the workspace. The wave whose
//           chunk holds the appended slot substitutes the new K row and, once its loads have
//           landed, writes the slot back to the cache as whole lines (the K lines it shares with
//           its neighbour slot, and, without the fused preparation, the slot's 8-slot V^T group).
//   values  one wave per 16-row d-block of V^T: the wave requests its first score row and its
//           whole V^T block (16 rows x the row's chunks, registers) right behind it, forms the
//           exact probabilities bf16(exp(s - m) / l) of its head while V is in flight (one LDS
//           exchange, one barrier that waits for LDS traffic only), then runs the value MFMAs.
//           Nothing is combined across workgroups.
// The probabilities are the single-launch kernels' (row max and row sum of the same bf16 scores),
// so the result differs from theirs only in the f32 order of the row sum.
//
// Workspace: scores bf16 [pairs][R][row_slots], row_slots = 512 (capacity <= 512) or 1024.

// Waves (32-slot K chunks) per scores workgroup. With the fused preparation every workgroup
// prepares the pair's q heads for itself, so 8 waves (two workgroups per 512-slot row) repeat it
// half as often as 4 (E2B decode step 4.484 -> 4.473 ms; 16 waves, one workgroup per row: 4.561).
constexpr int kTpWavesS = 8;
// Waves per values workgroup. Every workgroup forms the exact probabilities of the pair's heads for
// itself, so fewer, larger workgroups repeat less of that work: 8 waves (two workgroups per (b, kv
// head) at D = 256) for rows of up to 16 chunks, where the kernel holds 102 VGPRs (E2B decode step
// 4.86 -> 4.73 ms against 4 waves; 16 waves, one workgroup per pair: 4.50 -> 4.60 ms); 4 waves for
// longer rows, whose 152+ VGPRs would leave one 8-wave workgroup per CU.
template <int NCH>
constexpr int tp_waves_v() { return NCH <= 16 ? 8 : 4; }
constexpr int kTpMaxSlots = 1024;

__host__ __device__ inline int twopass_row_slots(int capacity) { return capacity <= 512 ? 512 : kTpMaxSlots; }

__host__ __device__ inline size_t twopass_workspace_bytes(int npairs, int R, int capacity) {
  return (size_t)npairs * R * twopass_row_slots(capacity) * 2;
}

// grid: pairs x parts, parts = ceil(ceil(capacity / 32) / kTpWavesS); wave w of part p takes chunk
// kTpWavesS * p + w.
//
// PREP: the launch also does g4_kv_append's work from the raw projection rows (G4DecodePrep). The
// waves of a workgroup prepare the pair's R query heads once (prep_head: g4_kv_append's own
// arithmetic) into LDS, where every wave reads its MFMA operand; in the workgroup whose chunks hold
// the appended slot, waves 0 and 1 also prepare the new K row (staged in LDS for the substitution,
// and stored to the cache) and the new V row (stored as the V^T column the values launch reads).
// The K chunk is requested before any of this, so the preparation runs while it is in flight.

// At most 128 registers up to head dim 256 (HIP's second launch bound is the minimum waves per SIMD:
// 4, two 8-wave workgroups per CU; the q operand is read from LDS slice by slice, so nothing spills:
// E2B decode step 4.76 -> 4.72 ms against 3 waves per SIMD). Without PREP the q rows are staged in
// LDS from q for the same reason (with the operand in registers, 138 registers and one workgroup
// per CU: 30.1 us for a full 512-slot ring at B = 256; at head dim 512, 36 bytes of spills). Head
// dim 512 holds 128 registers of K alone, so it takes no occupancy bound.
template <int D, bool PREP>
__global__ __launch_bounds__(kTpWavesS * 64, D <= 256 ? 4 : 1) void decode_bf16_tp_scores_kernel(G4DecodeArgs a, uint16_t* ws,
                                                                              int parts, int row_slots,
                                                                              G4DecodePrep pp) {
  constexpr int PER = D / 64;
  constexpr bool kQlds = PREP || D >= 256;  // the q operand read from LDS
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[kQlds ? 16 * D : 1];  // [R][D] (prepared) q
  __shared__ __attribute__((aligned(16))) uint16_t nk_lds[D];  // the (prepared) new K row, for the writer wave
  const int R = a.group;
  int pair, part;  // every part of a pair on one XCD
  xcd_item_part((int)blockIdx.x, a.batch * a.kv_heads, parts, pair, part);
  const int b = pair / a.kv_heads;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;
  KeyRange kr = key_range(a, b);
  if (PREP) kr.new_slot = pp.k_raw ? append_slot(a, kr.q) : -1;  // the append comes from the raw rows
  const int n_chunks = (kr.n_keys + 31) >> 5;
  const int chunk = part * kTpWavesS + w;
  const int new_chunk = kr.new_slot >= 0 ? (int)(kr.new_slot >> 5) : -1;
  const bool writer = new_chunk == chunk;  // the wave that scores the appended slot's chunk

  // PREP: the preparation's loads go out first (they return before the K chunk: vector loads
  // complete in issue order), so its arithmetic runs while the K chunk is in flight
  const int h = pair - b * a.kv_heads;
  const bool has_slot = PREP && pp.k_raw && new_chunk >= part * kTpWavesS && new_chunk < (part + 1) * kTpWavesS;
  const bool kv_wave = has_slot && w < 2;  // wave 0: the new K row, wave 1: the new V row
  PrepIn<true, D> pq, pkv;
  const uint16_t* qrow = reinterpret_cast<const uint16_t*>(pp.q_raw) + (int64_t)b * pp.in_row_stride;
  const float* rc = pp.rope_cos + (int64_t)b * D;
  const float* rs = pp.rope_sin + (int64_t)b * D;
  if constexpr (PREP) {
    if (w < R)
      prep_load<true, D, true>(pq, qrow + (int64_t)(h * R + w) * D, reinterpret_cast<const uint16_t*>(pp.q_norm_weight),
                               (pp.flags & G4_APPEND_ROPE_Q) != 0, rc, rs, lane);
    if (kv_wave)
      prep_load<true, D, true>(pkv,
                               reinterpret_cast<const uint16_t*>(w == 0 ? pp.k_raw : pp.v_raw) +
                                   (int64_t)b * pp.in_row_stride + (int64_t)h * D,
                               w == 0 ? reinterpret_cast<const uint16_t*>(pp.k_norm_weight) : nullptr,
                               w == 0 && (pp.flags & G4_APPEND_ROPE_K) != 0, rc, rs, lane);
  }
  // without PREP from D = 256: thread t's 16-byte pieces t, t + 512 of the pair's q rows, requested
  // ahead of the K chunk and stored to LDS once they land
  constexpr int kQPieces = kQlds && !PREP ? (16 * D / 8 + kTpWavesS * 64 - 1) / (kTpWavesS * 64) : 1;
  u32x4 qv[kQPieces];
  const int tid = threadIdx.x;
  if constexpr (kQlds && !PREP) {
#pragma unroll
    for (int j = 0; j < kQPieces; ++j) {
      const int t = tid + kTpWavesS * 64 * j;
      qv[j] = t < R * D / 8 ? load16(reinterpret_cast<const uint16_t*>(a.q) + (int64_t)pair * R * D + 8 * t)
                            : u32x4{0u, 0u, 0u, 0u};
    }
  }
  // without PREP: the writer wave's 16-byte pieces of the new K row (lane l < D / 8: dims 8 l ..
  // 8 l + 7), also requested ahead of the K chunk, so that the K substitution does not wait on a
  // load (with the new V row requested the same way: 52.2 -> 50.5 us per step for a full 512-slot
  // ring at B = 256 against loading the rows where they are used)
  u32x4 nkv = {0u, 0u, 0u, 0u};
  if (!PREP && writer && lane < D / 8) nkv = load16(reinterpret_cast<const uint16_t*>(a.new_k) + (int64_t)pair * D + 8 * lane);
  // ... and the appended slot's 8-slot group of the value cache (lane l: the 16-byte pieces of dims
  // l + 64 i) with the new value of each of those dims: the group is patched and stored back as
  // whole 16-byte pieces (whole lines) as soon as these land, before the scores (no load of this
  // launch reads the value cache; 50.5 -> 50.0 us against 2-byte stores of the column)
  constexpr int kVp = D / 64;
  u32x4 gv[kVp];
  uint16_t nvd[kVp];
  uint16_t* const cv_grp = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride +
                           (writer ? vt_index(kr.new_slot & ~(int64_t)7, 0, D) : 0);
  if (!PREP && writer) {
#pragma unroll
    for (int i = 0; i < kVp; ++i) {
      gv[i] = load16(cv_grp + 8 * (lane + 64 * i));
      nvd[i] = reinterpret_cast<const uint16_t*>(a.new_v)[(int64_t)pair * D + lane + 64 * i];
    }
  }
  u32x4 kv[2][D / 32];
  if (chunk < n_chunks) {
    const __amdgpu_buffer_rsrc_t rk =
        make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_k) + (int64_t)pair * a.slot_stride * D,
                  (uint32_t)a.slot_stride * D * 2u);
    load_k_chunk<D, true>(kv, rk, chunk << 5, col, grp);
  }
  if constexpr (PREP) {
    if (w < R) {
      prep_math<true, D>(pq, (pp.flags & G4_APPEND_NORM_Q) != 0, pp.q_norm_weight != nullptr,
                         (pp.flags & G4_APPEND_ROPE_Q) != 0, pp.eps);
      st_bf16<PER>(q_lds + w * D + lane * PER, pq.x);
    }
    for (int r = w + kTpWavesS; r < R; r += kTpWavesS) {  // more than one head per wave (R > 4)
      float x[PER];
      prep_head<true, D, true>(qrow + (int64_t)(h * R + r) * D, reinterpret_cast<const uint16_t*>(pp.q_norm_weight),
                               (pp.flags & G4_APPEND_NORM_Q) != 0, (pp.flags & G4_APPEND_ROPE_Q) != 0, rc, rs, pp.eps,
                               lane, x);
      st_bf16<PER>(q_lds + r * D + lane * PER, x);
    }
    if (kv_wave) {
      if (w == 0) {
        prep_math<true, D>(pkv, (pp.flags & G4_APPEND_NORM_K) != 0, pp.k_norm_weight != nullptr,
                           (pp.flags & G4_APPEND_ROPE_K) != 0, pp.eps);
        st_bf16<PER>(nk_lds + lane * PER, pkv.x);  // the writer wave stores it to the cache after its scores
      } else {
        prep_math<true, D>(pkv, (pp.flags & G4_APPEND_NORM_V) != 0, false, false, pp.eps);
        uint16_t* cv = reinterpret_cast<uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride;
#pragma unroll
        for (int e = 0; e < PER; ++e) cv[vt_index(kr.new_slot, lane * PER + e, D)] = (uint16_t)f32_to_bf16_bits(pkv.x[e]);
      }
    }
    wg_barrier();  // prepared q rows (and the new K row) are in LDS
  } else if constexpr (kQlds) {
#pragma unroll
    for (int j = 0; j < kQPieces; ++j) {
      const int t = tid + kTpWavesS * 64 * j;
      if (t < R * D / 8) reinterpret_cast<u32x4*>(q_lds)[t] = qv[j];
    }
    wg_barrier();  // q rows in LDS
  }

  if (!PREP && writer) {
    if (lane < D / 8) reinterpret_cast<u32x4*>(nk_lds)[lane] = nkv;  // read back by this wave only
    const int e = (int)(kr.new_slot & 7), wi = e >> 1;
#pragma unroll
    for (int i = 0; i < kVp; ++i) {
      u32x4 g = gv[i];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j == wi) g[j] = (e & 1) ? (g[j] & 0xffffu) | ((uint32_t)nvd[i] << 16) : (g[j] & 0xffff0000u) | nvd[i];
      *reinterpret_cast<u32x4*>(cv_grp + 8 * (lane + 64 * i)) = g;
    }
  }
  if (chunk < n_chunks) {
    bf16x8 qop[D / 32];
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      if constexpr (!kQlds) qop[s] = q_operand_global(a, pair, R, D, col, grp, s);
    }
    uint8_t mb;
    const bool ok = slot_valid_flat(a, b, kr, (chunk << 5) + (lane & 31), mb);
    const uint64_t vbits = __ballot(ok && mb != 0);
    if (writer && (!PREP || pp.k_raw)) {
      patch_k_sel<D>(kv, nk_lds, kr.new_slot, chunk << 5, col, grp);
      // the fused append's K row goes to the cache as soon as the chunk's loads have landed (no other
      // wave of the launch reads this chunk), as whole 128-byte lines: the new slot's pieces and its
      // line neighbour's (lanes col and col ^ 1 of the slot's half bb), both from the patched registers
      // (against the row's half lines stored after the scores: 50.0 -> 49.7 us per step for a full
      // 512-slot ring at B = 256; E2B decode step 4.431 -> 4.411 ms)
      const int r = (int)(kr.new_slot & 31);
      const int nc = ((r >> 3) << 2) | (r & 3), nbb = (r >> 2) & 1;
      if ((col >> 1) == (nc >> 1)) {
        unsigned char* ck = reinterpret_cast<unsigned char*>(a.cache_k_w) + (int64_t)pair * a.slot_stride * D * 2;
        const uint32_t base = (uint32_t)((chunk * (D / 32) * 2 + nbb) * 1024 + col * 64 + grp * 16);
        if (nbb) {  // (wave-uniform; static register indices)
#pragma unroll
          for (int s = 0; s < D / 32; ++s) *reinterpret_cast<u32x4*>(ck + base + 2048u * s) = kv[1][s];
        } else {
#pragma unroll
          for (int s = 0; s < D / 32; ++s) *reinterpret_cast<u32x4*>(ck + base + 2048u * s) = kv[0][s];
        }
      }
    }
    if constexpr (kQlds)
      score_to_lds_qlds<D>(kv, q_lds, vbits, ws + (int64_t)pair * R * row_slots, row_slots, chunk << 5, R, col, grp,
                           kBf16Min);
    else
      score_to_lds<D>(kv, qop, vbits, ws + (int64_t)pair * R * row_slots, row_slots, chunk << 5, R, col, grp,
                      kBf16Min);
  }
}

// Exact probabilities of head hh from its score row (lane owns slots 512 i + 8 lane .. +7, below
// `slots`) into LDS row hh; returns whether the row has no valid slot (then, with `store`, the
// row is the uniform bf16(1/capacity) over the capacity).
template <int NB>
__device__ __forceinline__ bool tp_probabilities(const u32x4 (&sv)[NB], int hh, bool store, uint16_t* sp,
                                                 int stride, int slots, int n_scanned, int capacity, int lane) {
  float e[NB][8];
  float m = kBf16Min;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int s0 = 512 * i + 8 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[i][2 * j] = s0 + 2 * j < n_scanned ? bf16_lo(sv[i][j]) : kBf16Min;
      e[i][2 * j + 1] = s0 + 2 * j + 1 < n_scanned ? bf16_hi(sv[i][j]) : kBf16Min;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, e[i][j]);
  }
  m = wave_max(m);
  const bool masked = m == kBf16Min;  // no valid slot in the row (the same for every head)
  if (!store) return masked;
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      e[i][j] = 512 * i + 8 * lane + j < n_scanned ? expf(e[i][j] - m) : 0.f;
      l += e[i][j];
    }
  }
  l = wave_sum(l);
  const float pu = round_bf16(1.0f / (float)capacity);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int s0 = 512 * i + 8 * lane;
    if (s0 < slots) {
      uint32_t pw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float p0, p1;
        if (masked) {
          p0 = s0 + 2 * j < capacity ? pu : 0.f;
          p1 = s0 + 2 * j + 1 < capacity ? pu : 0.f;
        } else {
          p0 = e[i][2 * j] / l;
          p1 = e[i][2 * j + 1] / l;
        }
        pw[j] = f32_to_bf16_bits(p0) | (f32_to_bf16_bits(p1) << 16);
      }
      *reinterpret_cast<u32x4*>(sp + hh * stride + s0) = u32x4{pw[0], pw[1], pw[2], pw[3]};
    }
  }
  return masked;
}

// LDS row stride (bf16 entries) of the values kernel's probabilities: 64 bytes of padding spread
// the R rows over the banks.
__host__ __device__ constexpr int tp_lds_stride(int nch) { return nch * 32 + 32; }

// grid: pairs x D / (16 tp_waves_v<NCH>()). NCH >= ceil(capacity / 32): V^T chunks held in registers.
template <int D, int NCH>
__global__ __launch_bounds__(tp_waves_v<NCH>() * 64) void decode_bf16_tp_values_kernel(G4DecodeArgs a, const uint16_t* ws,
                                                                              int row_slots) {
  constexpr int kTpWavesV = tp_waves_v<NCH>();
  constexpr int kParts = D / 16 / kTpWavesV;  // workgroups per pair
  static_assert(kParts >= 1 && kParts * kTpWavesV * 16 == D, "one 16-row d-block of V^T per wave");
  constexpr int NB = (NCH + 15) / 16;  // 512-slot blocks of a score row
  constexpr int kStride = tp_lds_stride(NCH);
  extern __shared__ float smem[];
  uint16_t* sp = reinterpret_cast<uint16_t*>(smem);  // [R][kStride] probabilities
  const int R = a.group;
  int pair, part;  // every part of a pair on one XCD
  xcd_item_part((int)blockIdx.x, a.batch * a.kv_heads, kParts, pair, part);
  const int b = pair / a.kv_heads;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int db = part * kTpWavesV + w;  // value dims [16*db, 16*db + 16)
  const KeyRange kr = key_range(a, b);
  const int n_chunks = (kr.n_keys + 31) >> 5;
  const int n_scanned = n_chunks << 5;
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(reinterpret_cast<const uint16_t*>(a.cache_vt) + (int64_t)pair * D * a.slot_stride,
                (uint32_t)a.slot_stride * D * 2u);
  const uint16_t* srow = ws + (int64_t)pair * R * row_slots;

  // requests: the score row of head w (head 0 for a wave without a head of its own: it needs only
  // the row's validity), then NCH V^T loads. All NCH are issued, so the wait for the score row
  // counts exactly the loads behind it; a chunk past the row's scanned ones is read at an offset
  // beyond the buffer resource's size, which returns zeros without a memory request.
  const int h0 = w < R ? w : 0;
  u32x4 sv[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    sv[i] = u32x4{0u, 0u, 0u, 0u};
    if (512 * i + 8 * lane < row_slots) sv[i] = load16(srow + h0 * row_slots + 512 * i + 8 * lane);
  }
  const uint32_t soff = 256u * db;  // value dims 16 db + col
  const uint32_t pair_bytes = (uint32_t)a.slot_stride * D * 2u;  // the resource's size: offsets from here read 0
  u32x4 vv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    vv[c] = buffer_load16_nt(rv, c < n_chunks ? vt_operand_bytes(4 * c + grp, col, D) : pair_bytes, soff);

  // exact probabilities: head w first; heads w + kTpWavesV, ... (more heads than waves) from rows loaded afterwards
  const bool all_masked = tp_probabilities<NB>(sv, w, w < R, sp, kStride, NCH * 32, n_scanned, a.capacity, lane);
  for (int hh = w + kTpWavesV; hh < R; hh += kTpWavesV) {
    u32x4 sh[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      sh[i] = u32x4{0u, 0u, 0u, 0u};
      if (512 * i + 8 * lane < row_slots) sh[i] = load16(srow + hh * row_slots + 512 * i + 8 * lane);
    }
    tp_probabilities<NB>(sh, hh, true, sp, kStride, NCH * 32, n_scanned, a.capacity, lane);
  }
  wg_barrier();  // probabilities are in LDS (the V^T loads stay in flight)

  floatx4 oacc = {0.f, 0.f, 0.f, 0.f}, oacc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NCH; c += 2) {
    if (c < n_chunks)
      oacc = mfma16x16x32(as_bf16x8(vv[c]), prob_operand(sp, kStride, (c << 5) + 8 * grp, R, col), oacc);
    if (c + 1 < n_chunks)
      oacc1 = mfma16x16x32(as_bf16x8(vv[c + 1]), prob_operand(sp, kStride, ((c + 1) << 5) + 8 * grp, R, col), oacc1);
  }
  oacc += oacc1;
  // a fully masked row averages every slot below the capacity, including ones never scanned
  if (all_masked) {
    const int cap_chunks = (a.capacity + 31) >> 5;
    for (int c = n_chunks; c < cap_chunks; ++c) {
      const u32x4 v = buffer_load16_nt(rv, vt_operand_bytes(4 * c + grp, col, D), soff);
      oacc = mfma16x16x32(as_bf16x8(v), prob_operand(sp, kStride, (c << 5) + 8 * grp, R, col), oacc);
    }
  }
  // lane (grp, col < R) holds O^T[d = 16*db + 4*grp + j][head col]
  if (col < R) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)pair * R + col) * D;
    const uint32_t w0 = f32_to_bf16_bits(oacc[0]) | (f32_to_bf16_bits(oacc[1]) << 16);
    const uint32_t w1 = f32_to_bf16_bits(oacc[2]) | (f32_to_bf16_bits(oacc[3]) << 16);
    *reinterpret_cast<uint2*>(orow + 16 * db + 4 * grp) = make_uint2(w0, w1);
  }
}
