// The LM head with the sampler in its epilogue (g4_lm_head_sample): logits = x . embed^T for the
// decode batch (bf16 in, f32 accumulation, bf16 logits: model.py:676-680 with the tied embedding),
// then _sample_token (sampler.py:145-183) without the logits ever reaching HBM. With token_out NULL
// it is the plain LM head (bf16 logits into logits_out).
//
// One persistent grid of two workgroups per CU. A workgroup owns all M <= 256 rows and walks its
// vocab tiles of 128 columns (tile t, t + grid, ...). Per tile: the GEMM over K in stages of 32
// (x 256 x 32 and embed 128 x 32 DMA'd into a 3-slot LDS ring, two stages in flight; the ring runs
// on across tiles, so the next tile's first stages load during this tile's epilogue), then the
// epilogue on the accumulators in registers: bf16 rounding, the soft-cap, the running max / sum of
// the full-vocab log-softmax, Gumbel noise from JAX's threefry stream and the running argmax.
// The epilogue is VALU work (the threefry rounds dominate); the GEMM is weight streaming and MFMA,
// so the two workgroups of a CU overlap one's epilogue with the other's GEMM.
//
// Wave w owns rows [64 w, 64 w + 64) x the tile's 128 columns: MFMA v_mfma_f32_16x16x32_bf16 with
// A = 16 embed rows (vocab columns), B = 16 x rows; lane (grp, col) accumulates
// logits[64 w + 16 rb + col][16 cb + 4 grp + j]. The lane keeps one running state per row it holds
// (rb = 0..3) across the workgroup's tiles, visiting its columns in increasing order, so a strict
// comparison keeps the first of equal scores. At the end the 4 lanes of a row merge (column order
// decides ties) and the workgroup writes one state per row; a combine kernel merges the
// workgroups' states in workgroup order, writes the token and its log-probability, and splits the
// loop key.
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

#include "g4_sample_common.h"  // threefry2x32, Gumbel noise

constexpr int kLhRows = 256;  // rows per workgroup (all of them)
constexpr int kLhCols = 128;  // vocab columns per tile
constexpr int kLhKT = 32;     // K per stage (one MFMA)
constexpr int kLhSlots = 3;   // LDS ring slots: two stages in flight
constexpr int kLhThreads = 256;
constexpr int kLhXBytes = kLhRows * kLhKT * 2;   // 16 KiB: 256 rows x 64 bytes
constexpr int kLhWBytes = kLhCols * kLhKT * 2;   // 8 KiB: 128 rows x 64 bytes
constexpr int kLhSlotBytes = kLhXBytes + kLhWBytes;
constexpr int kLhDmaPerWave = (kLhRows + kLhCols) / 16 / 4;  // 16-row DMA groups per wave and stage: 6
constexpr int kLhWgPerCu = 2;

int g_lh_grid[kMaxDevices];  // persistent grid size per device (2 x CUs), set by setup_lm_head

// Per-workgroup row states in the workspace: [grid][256] of each field.
struct LhStates {
  float* m;
  float* s;
  float* best;
  float* bx;  // the capped logit of the best column (for the log-probability)
  int* idx;
};

__host__ __device__ inline LhStates lh_states(void* ws, int grid) {
  const size_t n = (size_t)grid * kLhRows;
  LhStates st;
  st.m = reinterpret_cast<float*>(ws);
  st.s = st.m + n;
  st.best = st.s + n;
  st.bx = st.best + n;
  st.idx = reinterpret_cast<int*>(st.bx + n);
  return st;
}

struct LhState {
  float m, s, best, bx;
  int idx;
};

__device__ __forceinline__ void lh_merge(LhState& a, const LhState& b) {
  if (b.m > a.m) {
    a.s = a.s * expf(a.m - b.m) + b.s;
    a.m = b.m;
  } else if (b.m > kF32Min) {
    a.s += b.s * expf(b.m - a.m);
  }
  if (beats(b.best, b.idx, a.best, a.idx)) {  // ties and NaNs: the first column (argmax)
    a.best = b.best;
    a.bx = b.bx;
    a.idx = b.idx;
  }
}

__device__ __forceinline__ LhState lh_shfl(const LhState& x, int mask) {
  LhState y;
  y.m = __shfl_xor(x.m, mask, 64);
  y.s = __shfl_xor(x.s, mask, 64);
  y.best = __shfl_xor(x.best, mask, 64);
  y.bx = __shfl_xor(x.bx, mask, 64);
  y.idx = __shfl_xor(x.idx, mask, 64);
  return y;
}

// DMA of one stage (K offset k0, vocab tile n0) into `slot`: groups of 16 rows x 64 bytes (one
// instruction: 64 lanes x 16 bytes landing at lane * 16). Within a group, row r's 16-byte piece p
// sits at 16-byte slot 4 r + (p ^ ((r >> 1) & 3)), so the 8 rows of an operand read's phase fall on
// 8 different 16-byte bank groups; lane l fetches the piece that belongs at slot l (row l / 4, the
// row's four pieces from the same 64-byte segment). Groups 0..15 are x rows, 16..23 embed rows;
// wave w moves groups w, w + 4, ..., w + 20. x rows >= M read beyond the resource: zeros.
__device__ __forceinline__ int lh_swz(int r) { return (r >> 1) & 3; }

__device__ __forceinline__ void lh_dma(unsigned char* __restrict__ slot, __amdgpu_buffer_rsrc_t rx,
                                       __amdgpu_buffer_rsrc_t rw, int K, int k0, int n0, int w, int lane) {
  const int rl = lane >> 2, piece = (lane & 3) ^ lh_swz(lane >> 2);
#pragma unroll
  for (int i = 0; i < kLhDmaPerWave; ++i) {
    const int g = w + 4 * i;
    const bool is_x = g < kLhRows / 16;
    const int row = is_x ? 16 * g + rl : n0 + 16 * (g - kLhRows / 16) + rl;
    const uint32_t off = (uint32_t)(row * K + k0 + 8 * piece) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(is_x ? rx : rw,
                                             (__attribute__((address_space(3))) void*)(slot + g * 1024), 16, off, 0,
                                             0, 0);
  }
}

// One stage's MFMAs for wave w: 4 x-row blocks (B operands) x 8 embed-row blocks (A operands).
__device__ __forceinline__ void lh_compute(uint32_t slot, floatx4 (&acc)[4][8], int w, int col, int grp) {
  // row 16 b + col of a part, piece grp: group b, slot 4 col + (grp ^ swz(col))
  const uint32_t in_group = (uint32_t)col * 64u + (uint32_t)(grp ^ lh_swz(col)) * 16u;
  const uint32_t xs = slot + (uint32_t)(4 * w) * 1024u + in_group;
  const uint32_t ws = slot + (uint32_t)kLhXBytes + in_group;
  u32x4 b[4], a[8];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) b[rb] = lds_read16(xs + 1024u * rb);
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) a[cb] = lds_read16(ws + 1024u * cb);
  __asm__ volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]),
                     "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]));
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) acc[rb][cb] = mfma16x16x32(as_bf16x8(a[cb]), as_bf16x8(b[rb]), acc[rb][cb]);
}

// The epilogue of four consecutive columns n .. n + 3 of one row: bf16 rounding (the logits), the
// optional logits store, the soft-cap, the running max / sum and the running argmax of the scores.
// UNIT_T: temperature 1, no division (the compiler would otherwise divide every logit and select).
template <bool SAMPLE, bool GREEDY, bool UNIT_T>
__device__ __forceinline__ void lh_epilogue(floatx4 v, LhState& sr, int row, int n, const G4LmHeadSampleArgs& a,
                                            const CapTable& ct, uint32_t k0, uint32_t k1) {
  uint32_t bits[4];
  float x[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bits[j] = f32_to_bf16_bits(v[j]);
    x[j] = bf16_bits_to_f32(bits[j]);
  }
  if (a.logits_out) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.logits_out) + (int64_t)row * a.vocab + n;
    *reinterpret_cast<uint2*>(dst) = make_uint2(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16));
  }
  if constexpr (SAMPLE) {
    if (a.softcap > 0.f) {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = capped(bits[j], ct);
    }
    const float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    if (mx > sr.m) {  // a new running max: rescale the sum (else the factor would be exactly 1)
      sr.s *= expf(sr.m - mx);
      sr.m = mx;
    }
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) sum += expf(x[j] - sr.m);
    sr.s += sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float score = x[j];
      if constexpr (!GREEDY) {
        const float t = UNIT_T ? x[j] : x[j] / a.temperature;
        score = t + gumbel(k0, k1, (uint64_t)row * (uint64_t)a.vocab + (uint64_t)(n + j));
      }
      if (takes_best(score, sr.best)) {
        sr.best = score;
        sr.bx = x[j];
        sr.idx = n + j;
      }
    }
  }
}

// SAMPLE: run the sampler epilogue (else only the bf16 logits are written); GREEDY: no noise;
// UNIT_T: temperature 1.
template <bool SAMPLE, bool GREEDY, bool UNIT_T = false>
__global__ __launch_bounds__(kLhThreads, kLhWgPerCu) void lm_head_kernel(G4LmHeadSampleArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char ring[kLhSlots][kLhSlotBytes];
  __shared__ uint16_t cap_tab[SAMPLE ? kCapTableEntries : 1];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int K = a.hidden, V = a.vocab, M = a.batch;
  const int nst = K / kLhKT;
  const int n_tiles = V / kLhCols;
  const int grid = (int)gridDim.x;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.embed, (uint32_t)V * (uint32_t)K * 2u);
  const uint32_t ring0 = lds_addr(&ring[0][0]);

  uint32_t k0 = 0u, k1 = 0u;  // the sample key
  if constexpr (SAMPLE && !GREEDY) {
    if (a.split_key) {  // sample_key = split(key)[1] = threefry2x32(key, (0, 1))
      k1 = 1u;
      threefry2x32(a.key[0], a.key[1], k0, k1);
    } else {
      k0 = a.key[0];
      k1 = a.key[1];
    }
  }
  LhState st[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) st[rb] = LhState{kF32Min, 0.f, -INFINITY, 0.f, 0x7fffffff};
  const CapTable ct = cap_table(cap_tab, a.softcap);
  if (SAMPLE && a.softcap > 0.f) {  // the soft-cap table, complete before any DMA is issued
    cap_table_fill(cap_tab, a.softcap, threadIdx.x, kLhThreads);
    __syncthreads();
  }

  // the ring's stage sequence runs over every (tile, k stage) of this workgroup; stage q of the
  // sequence sits in slot q % 3. Stages past the last tile re-read stage 0 of the last tile (an L2
  // hit), so every wave issues the same number of DMAs per step.
  const int my_tiles = blockIdx.x < n_tiles ? (n_tiles - 1 - (int)blockIdx.x) / grid + 1 : 0;
  const int total = my_tiles * nst;
  auto issue = [&](int q) {
    const int qq = q < total ? q : (total > 0 ? total - nst : 0);
    const int t = (int)blockIdx.x + (qq / nst) * grid;
    lh_dma(&ring[q % kLhSlots][0], rx, rw, K, (qq % nst) * kLhKT, t * kLhCols, w, lane);
  };
  if (total > 0) {
    issue(0);
    issue(1);
  }
  int q = 0;
  for (int it = 0; it < my_tiles; ++it) {
    const int n0 = ((int)blockIdx.x + it * grid) * kLhCols;
    floatx4 acc[4][8];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) acc[rb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nst; ++s, ++q) {
      // this wave's DMAs of stage q have landed (those of q + 1 may not have), then every wave's;
      // every wave is also past stage q - 1, whose slot the DMAs of q + 2 refill
      __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kLhDmaPerWave) : "memory");
      issue(q + 2);
      lh_compute(ring0 + (uint32_t)(q % kLhSlots) * kLhSlotBytes, acc, w, col, grp);
    }

    // ---- epilogue: lane (grp, col) holds logits[64 w + 16 rb + col][n0 + 16 cb + 4 grp + j] ----------
    // The cb loop stays a loop (code size): each iteration takes block acc[rb][0] and rotates the
    // row's eight blocks by one, so every register index is static.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row = 64 * w + 16 * rb + col;
      if (row < M) {
#pragma unroll 1
        for (int cb = 0; cb < 8; ++cb) {
          const floatx4 v = acc[rb][0];
#pragma unroll
          for (int i = 0; i < 7; ++i) acc[rb][i] = acc[rb][i + 1];
          acc[rb][7] = v;
          lh_epilogue<SAMPLE, GREEDY, UNIT_T>(v, st[rb], row, n0 + 16 * cb + 4 * grp, a, ct, k0, k1);
        }
      }
    }
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the trailing DMAs land before the wave ends

  if constexpr (SAMPLE) {
    // the 4 lanes of a row (grp 0..3) merge; lane grp = 0 writes the workgroup's state of the row
    const LhStates ws = lh_states(a.workspace, grid);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      LhState x = st[rb];
      lh_merge(x, lh_shfl(x, 16));
      lh_merge(x, lh_shfl(x, 32));
      const int row = 64 * w + 16 * rb + col;
      if (grp == 0 && row < M) {
        const size_t i = (size_t)blockIdx.x * kLhRows + row;
        ws.m[i] = x.m;
        ws.s[i] = x.s;
        ws.best[i] = x.best;
        ws.bx[i] = x.bx;
        ws.idx[i] = x.idx;
      }
    }
  }
}

// One workgroup per row: merge the workgroups' states in workgroup order (each thread a strided
// run, then a fixed reduction tree), write the token and log(softmax(capped logits))[token]; block
// 0 then splits the loop key (every workgroup of the LM head kernel has read it).
constexpr int kCombineThreads = 256;

__global__ __launch_bounds__(kCombineThreads) void lm_head_combine_kernel(G4LmHeadSampleArgs a, int grid) {
  __shared__ LhState red[kCombineThreads];
  // Workgroups are dealt to the 8 XCDs round robin (blockIdx mod 8). The states of consecutive rows
  // share cache lines (32 rows per 128-byte line of each array), so each XCD takes a contiguous
  // block of batch / 8 rows: a line is fetched into one XCD's L2, not into all eight.
  const int wg = (int)blockIdx.x;
  const int row = a.batch % 8 == 0 ? (wg & 7) * (a.batch >> 3) + (wg >> 3) : wg;
  const LhStates ws = lh_states(a.workspace, grid);
  LhState st = {kF32Min, 0.f, -INFINITY, 0.f, 0x7fffffff};
  // states g = tid, tid + 256, ... merged in that order; two of them are requested before either
  // is merged (one round trip for the 512-workgroup grid of 256 CUs)
  for (int g0 = threadIdx.x; g0 < grid; g0 += 2 * kCombineThreads) {
    LhState v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int g = g0 + u * kCombineThreads;
      if (g < grid) {
        const size_t i = (size_t)g * kLhRows + row;
        v[u] = LhState{ws.m[i], ws.s[i], ws.best[i], ws.bx[i], ws.idx[i]};
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (g0 + u * kCombineThreads < grid) lh_merge(st, v[u]);
  }
  // tree: at level h thread t < h merges thread t + h (h = 128, 64 through LDS, then 32 .. 1 by
  // shuffles within wave 0, where lane t reads lane t ^ h = t + h)
  red[threadIdx.x] = st;
  __syncthreads();
  for (int h = kCombineThreads / 2; h >= 64; h >>= 1) {
    if ((int)threadIdx.x < h) {
      LhState x = red[threadIdx.x];
      lh_merge(x, red[threadIdx.x + h]);
      red[threadIdx.x] = x;
    }
    __syncthreads();
  }
  if (threadIdx.x < 64) {
    LhState t = red[threadIdx.x];
#pragma unroll
    for (int h = 32; h >= 1; h >>= 1) {
      const LhState y = lh_shfl(t, h);
      if ((int)threadIdx.x < h) lh_merge(t, y);
    }
    if (threadIdx.x != 0) return;
    // only a row whose every score is -inf keeps no best: clamp the token into the vocab
    const int token = t.idx < 0 ? 0 : (t.idx >= a.vocab ? a.vocab - 1 : t.idx);
    a.token_out[row] = token;
    a.logp_out[row] = (t.bx - t.m) - logf(t.s);
    if (row == 0 && a.key && a.split_key) {  // key <- split(key)[0] = threefry2x32(key, (0, 0))
      uint32_t x0 = 0u, x1 = 0u;
      threefry2x32(a.key[0], a.key[1], x0, x1);
      a.key[0] = x0;
      a.key[1] = x1;
    }
  }
}

int lh_grid(const G4LmHeadSampleArgs& a, int dev) {
  const int n_tiles = a.vocab / kLhCols;
  const int g = g_lh_grid[dev];
  return g < n_tiles ? g : n_tiles;
}

}  // namespace

// The persistent grid of this device: two workgroups per CU (run once per device by device_setup).
// Without a CU count the grid stays 0 and only g4_lm_head_sample reports it.
int setup_lm_head(int device) {
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, device) != hipSuccess || p.multiProcessorCount <= 0) {
    (void)hipGetLastError();
    g_lh_grid[device] = 0;
    return G4_OK;
  }
  g_lh_grid[device] = kLhWgPerCu * p.multiProcessorCount;
  return G4_OK;
}

}  // namespace g4

extern "C" size_t g4_lm_head_sample_workspace_size(const G4LmHeadSampleArgs* args) {
  using namespace g4;
  if (!args || !args->token_out) return 0;
  int dev = 0;
  if (device_setup(&dev) != G4_OK) return 0;
  return (size_t)lh_grid(*args, dev) * kLhRows * 5u * 4u;
}

extern "C" int g4_lm_head_sample(const G4LmHeadSampleArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_lm_head_sample: args is NULL");
  const G4LmHeadSampleArgs& a = *args;
  if (a.batch <= 0 || a.batch > kLhRows)
    return fail(G4_ERR_UNSUPPORTED, "g4_lm_head_sample: batch %d (1..%d)", a.batch, kLhRows);
  if (a.vocab <= 0 || a.vocab % kLhCols)
    return fail(G4_ERR_UNSUPPORTED, "g4_lm_head_sample: vocab %d (a multiple of %d)", a.vocab, kLhCols);
  if (a.hidden <= 0 || a.hidden % kLhKT)
    return fail(G4_ERR_UNSUPPORTED, "g4_lm_head_sample: hidden %d (a multiple of %d)", a.hidden, kLhKT);
  if ((int64_t)a.vocab * a.hidden * 2 >= (int64_t)1 << 32)
    return fail(G4_ERR_UNSUPPORTED, "g4_lm_head_sample: embed beyond 4 GiB");
  if (!a.x || !a.embed) return fail(G4_ERR_INVALID, "g4_lm_head_sample: NULL x / embed");
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) || (reinterpret_cast<uintptr_t>(a.embed) & 15) ||
      (reinterpret_cast<uintptr_t>(a.logits_out) & 7))
    return fail(G4_ERR_INVALID, "g4_lm_head_sample: x / embed need 16-byte and logits_out 8-byte alignment");
  const bool sample = a.token_out != nullptr;
  if (!sample && !a.logits_out) return fail(G4_ERR_INVALID, "g4_lm_head_sample: neither token_out nor logits_out");
  if (sample && !a.logp_out) return fail(G4_ERR_INVALID, "g4_lm_head_sample: token_out without logp_out");
  if (!(a.softcap >= 0.f)) return fail(G4_ERR_INVALID, "g4_lm_head_sample: softcap must be >= 0");
  const bool greedy = !(a.temperature > 0.f);
  if (sample && !greedy && !a.key) return fail(G4_ERR_INVALID, "g4_lm_head_sample: sampling needs the device key");
  if (a.split_key != 0 && a.split_key != 1) return fail(G4_ERR_INVALID, "g4_lm_head_sample: split_key %d", a.split_key);
  int dev = 0;
  if (int rc = device_setup(&dev)) return rc;
  const int grid = lh_grid(a, dev);
  if (grid <= 0)
    return fail(G4_ERR_LAUNCH, "g4_lm_head_sample: the CU count of device %d could not be read at set-up", dev);
  if (sample) {
    const size_t need = (size_t)grid * kLhRows * 5u * 4u;
    if (!a.workspace || a.workspace_bytes < need)
      return fail(G4_ERR_WORKSPACE, "g4_lm_head_sample: needs %zu B of workspace (have %zu)", need,
                  a.workspace ? a.workspace_bytes : (size_t)0);
    if (reinterpret_cast<uintptr_t>(a.workspace) & 3)
      return fail(G4_ERR_INVALID, "g4_lm_head_sample: workspace needs 4-byte alignment");
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!sample)
    hipLaunchKernelGGL((lm_head_kernel<false, true>), dim3((unsigned)grid), dim3(kLhThreads), 0, st, a);
  else if (greedy)
    hipLaunchKernelGGL((lm_head_kernel<true, true>), dim3((unsigned)grid), dim3(kLhThreads), 0, st, a);
  else if (a.temperature == 1.0f)
    hipLaunchKernelGGL((lm_head_kernel<true, false, true>), dim3((unsigned)grid), dim3(kLhThreads), 0, st, a);
  else
    hipLaunchKernelGGL((lm_head_kernel<true, false>), dim3((unsigned)grid), dim3(kLhThreads), 0, st, a);
  if (int rc = check_launch("g4_lm_head_sample")) return rc;
  if (!sample) return G4_OK;
  hipLaunchKernelGGL(lm_head_combine_kernel, dim3((unsigned)a.batch), dim3(kCombineThreads), 0, st, a, grid);
  return check_launch("g4_lm_head_sample (combine)");
}
