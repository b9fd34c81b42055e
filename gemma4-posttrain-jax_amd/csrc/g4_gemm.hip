// Decode-step projection GEMM (g4_linear_bf16): Y[M, N] = X[M, K] . W[N, K]^T, bf16 in, f32
// accumulation, bf16 out, for the rollout's decode batch (M <= 256 rows). Replaces the dense
// projections of forward_attention / forward_mlp (model.py:463-482, 393-396, 500) at S = 1.
//
// At M = 256 the projection is a stream of the weight matrix: every weight byte is used by all
// 256 rows once. A workgroup owns 128 rows x 128 columns of the output (the two row halves of a
// column tile on one XCD, so W is read from HBM once; 256 rows x 64 columns below 129 rows), and
// X (shared by every workgroup) comes from L2. K is walked in stages of 64: the X and W stages are
// DMA'd into a 4-deep LDS ring (buffer_load ... lds), three stages in flight while the fourth is
// multiplied.
//
// LDS layout of a stage: groups of 8 rows x 128 bytes (one DMA instruction: 64 lanes x 16 bytes,
// 8 full 128-byte lines of the row-major operand); within a group, row r's
// 16-byte piece kc sits at slot kc ^ r, so the 16 rows an MFMA operand read touches fall on
// different banks. Each lane DMAs the piece that belongs at its slot.
//
// MFMA v_mfma_f32_16x16x32_bf16 with A = 16 rows of W (output columns) and B = 16 rows of X
// (output rows): lane (grp, col) accumulates Y[m = 16 rb + col][n = 16 cb + 4 grp .. + 3], four
// consecutive outputs of one row. Each of the 8 waves owns a 64 x 32 block of the 128 x 128 or
// 256 x 64 tile (4 x 2 accumulator blocks).
//
// Split-K (ksplit > 1): a workgroup of split s covers K range s; partial sums go to an f32
// workspace [ksplit][M][N] and a second kernel adds them in split order and rounds to bf16, or,
// with no y given, they are left there for a consumer that adds them itself
// (g4_residual_norm_splitk, the residual norm after the MLP's down projection).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kGemmRows = 256;  // M rows at most
constexpr int kGemmKT = 64;     // K per stage
constexpr int kGroupBytes = 1024;  // 8 rows x 128 B

// A workgroup's tile: TR rows x TC columns (TR / 64 waves along the rows, TC / WCOLS along the
// columns). TR = 256: all rows, 64 columns (X re-read once per 64 columns). TR = 128: half
// the rows, 128 columns (per CU 1/4 less X + W traffic; the two row halves of a column tile go to
// one XCD, so the second read of its W is an L2 hit).
// Every wave owns 64 x 32 outputs: 8 waves per workgroup, two per SIMD, so one's MFMAs run while the
// other waits on its stage; each output keeps the same K order as with 4 waves of 64 x 64, so the
// results are identical. TR = 128 (M 256): gate/up 31.4-33.2 -> 29.5-31.1 us, down 18.2-18.6 ->
// 17.7-18.0 us, E2B decode step 4.542 -> 4.505 ms; TR = 256 (M 128 / 64): gate/up 29.3-31.3 ->
// 25.9-27.5 / 28.8-29.7 -> 25.4-26.4 us, down 16.2-16.5 -> 14.2-14.9 / 15.0 -> 12.9-13.2 us.
template <int TR>
struct GemmTile {
  static constexpr int TC = 16384 / TR;
  static constexpr int WR = TR / 64;                  // waves along the rows
  static constexpr int WCOLS = 32;                    // columns per wave
  static constexpr int CB = WCOLS / 16;               // 16-column MFMA blocks per wave
  static constexpr int WAVES = WR * (TC / WCOLS);
  static constexpr int THREADS = WAVES * 64;
  static constexpr int XG = TR / 8;   // 8-row groups of X per stage
  static constexpr int WG = TC / 8;   // of W
  static constexpr int DMA = (XG + WG) / WAVES;  // DMA instructions per wave and stage
  static constexpr int STAGE = (XG + WG) * kGroupBytes;        // 40 KiB (TR 256) / 32 KiB (TR 128)
  static_assert(TR == 256 || TR == 128, "tile rows");
  static_assert((XG + WG) % WAVES == 0 && WAVES * 64 <= 1024, "every wave issues the same DMA count");
};

// First weight row of W group j (8 rows) of column tile `tile`. Plain: rows tile * TC + 8 j. Gated
// GELU: each WCOLS-column wave slice holds the WCOLS / 2 gate rows and the WCOLS / 2 up rows of the
// same outputs (gate rows of output o at o, up rows at half + o), tile * TC / 2 outputs before this
// tile.
template <int TC, int WCOLS>
__device__ __forceinline__ int gemm_wrow(bool gelu, int half, int tile, int j) {
  if (!gelu) return tile * TC + 8 * j;
  constexpr int GS = WCOLS / 8;  // 8-row groups per wave slice: the first GS / 2 are gate rows
  const int o = tile * (TC / 2) + (WCOLS / 2) * (j / GS) + 8 * (j % (GS / 2));
  return j % GS < GS / 2 ? o : half + o;
}

// DMA of the stage at K offset k0 into `buf`: wave w moves groups w, w + WAVES, ... of X then of W.
// Lane l of a group instruction takes row 8 g + l / 8 and the 16-byte piece (l % 8) ^ (row % 8) of
// its 128-byte K slice. Past the last stage every load reads beyond its resource (zeros, no memory
// request), so every wave always issues the same number of loads per stage.
template <int TR>
__device__ __forceinline__ void gemm_dma(unsigned char* __restrict__ buf, __amdgpu_buffer_rsrc_t rx,
                                         __amdgpu_buffer_rsrc_t rw, int K, int k0, bool live, uint32_t oob_x,
                                         uint32_t oob_w, int w, int lane, int m0, bool gelu, int half, int tile) {
  using T = GemmTile<TR>;
  const int rl = lane >> 3;        // row within the group
  const int kc = (lane & 7) ^ rl;  // 16-byte piece this lane fetches (row % 8 == rl)
#pragma unroll
  for (int i = 0; i < T::DMA; ++i) {
    const int g = w + T::WAVES * i;  // groups 0..XG-1: X, then W
    const bool is_x = g < T::XG;
    const int row = is_x ? m0 + 8 * g + rl : gemm_wrow<T::TC, T::WCOLS>(gelu, half, tile, g - T::XG) + rl;
    const uint32_t off = (uint32_t)(row * K + k0 + 8 * kc) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(is_x ? rx : rw,
                                             (__attribute__((address_space(3))) void*)(buf + g * kGroupBytes), 16,
                                             live ? off : (is_x ? oob_x : oob_w), 0, 0, 0);
  }
}

// LDS byte offset of the 16-byte MFMA operand piece kc of row `row` (within the X or W part of a
// stage).
__device__ __forceinline__ uint32_t gemm_operand_at(uint32_t part, int row, int kc) {
  const int r = row & 7;
  return part + (uint32_t)((row >> 3) * kGroupBytes + (8 * r + (kc ^ r)) * 16);
}

// The operand reads are issued as ds_read_b128 in inline assembly (lds_read16) and waited for
// explicitly (lgkmcnt, tied to the eight operand registers). Read through C++, the compiler cannot
// tell the stage being multiplied from the stages the DMA is still filling, and at some steps of
// the ring waited for every DMA in flight (vmcnt(0)); the stage's own DMAs are already covered by
// the s_waitcnt vmcnt + s_barrier that starts each step.
// Wave (wr, wc) multiplies rows [64 wr, 64 wr + 64) of the X part by rows [WCOLS wc, WCOLS wc +
// WCOLS) of the W part.
template <int TR>
__device__ __forceinline__ void gemm_compute(const unsigned char* __restrict__ buf,
                                             floatx4 (&acc)[4][GemmTile<TR>::CB], int wr, int wc, int col, int grp) {
  constexpr int CB = GemmTile<TR>::CB, WCOLS = GemmTile<TR>::WCOLS;
  const uint32_t xs = lds_addr(buf);
  const uint32_t ws = xs + GemmTile<TR>::XG * kGroupBytes;
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    static_assert(CB == 2, "operand wait list");
    u32x4 a[CB], b[4];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) a[cb] = lds_read16(gemm_operand_at(ws, WCOLS * wc + 16 * cb + col, 4 * kh + grp));
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) b[rb] = lds_read16(gemm_operand_at(xs, 64 * wr + 16 * rb + col, 4 * kh + grp));
    __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = mfma16x16x32(as_bf16x8(a[cb]), as_bf16x8(b[rb]), acc[rb][cb]);
  }
}

struct GemmLoop {
  __amdgpu_buffer_rsrc_t rx, rw;
  int K, kbeg, nst;
  uint32_t oob_x, oob_w;
  int w, lane, col, grp, wr, wc, m0, half, tile;
  bool gelu;
};

// One pipeline step: stage s is in `cur` (stages s + 1, s + 2 in flight); stage s + 3 is
// requested into `fre` (the buffer of stage s - 1, which every wave has finished with) after the
// stage's MFMAs are issued, so a DMA issue that waits for room in the memory queue does not hold
// them back (down projection 19.3 -> 18.6 us).
template <int TR>
__device__ __forceinline__ void gemm_step(const unsigned char* __restrict__ cur, unsigned char* __restrict__ fre,
                                          floatx4 (&acc)[4][GemmTile<TR>::CB], const GemmLoop& L, int s) {
  // this wave's DMAs of stage s have landed (stages s + 1, s + 2 may not have), then every wave's
  __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * GemmTile<TR>::DMA) : "memory");
  gemm_compute<TR>(cur, acc, L.wr, L.wc, L.col, L.grp);
  gemm_dma<TR>(fre, L.rx, L.rw, L.K, L.kbeg + (s + 3) * kGemmKT, s + 3 < L.nst, L.oob_x, L.oob_w, L.w, L.lane, L.m0,
               L.gelu, L.half, L.tile);
}

// Work units (column tile, K split), each covered by n_halves = ceil(M / TR) workgroups (row
// halves). Workgroups are dealt to the 8 XCDs round robin (i mod 8); when the unit count is a
// multiple of 8, workgroup i takes unit 8 (j / n_halves) + i mod 8 and half j mod n_halves
// (j = i / 8), so all halves of a unit share an XCD (one HBM read of its W) and, with ksplit
// dividing 8, every XCD works on one K split, whose slice of X its L2 then holds for all its
// column tiles. The unit is (tile u / ksplit, split u mod ksplit). K / ksplit must be a multiple
// of 64.
template <int TR>
__global__ __launch_bounds__(GemmTile<TR>::THREADS) void linear_bf16_kernel(G4LinearArgs a, float* partials) {
  using T = GemmTile<TR>;
  __shared__ __attribute__((aligned(1024))) unsigned char b0[T::STAGE], b1[T::STAGE], b2[T::STAGE], b3[T::STAGE];
  GemmLoop L;
  L.lane = threadIdx.x & 63;
  L.w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  L.col = L.lane & 15;
  L.grp = L.lane >> 4;
  L.wr = L.w % T::WR;
  L.wc = L.w / T::WR;
  const int n_halves = (a.m + TR - 1) / TR;
  const int n_units = a.n / T::TC * a.ksplit;
  const int i = (int)blockIdx.x;
  int unit, hf;
  if (n_units % 8 == 0) {
    const int j = i >> 3;
    unit = 8 * (j / n_halves) + (i & 7);
    hf = j % n_halves;
  } else {
    unit = i / n_halves;
    hf = i % n_halves;
  }
  L.tile = unit / a.ksplit;
  const int split = unit - L.tile * a.ksplit;
  L.m0 = hf * TR;
  const int n0 = L.tile * T::TC;
  L.K = a.k;
  const int kper = L.K / a.ksplit;
  L.kbeg = split * kper;
  L.nst = kper / kGemmKT;
  const uint32_t xbytes = (uint32_t)a.m * (uint32_t)L.K * 2u;  // rows >= M read as zeros
  const uint32_t wbytes = (uint32_t)a.n * (uint32_t)L.K * 2u;
  L.oob_x = xbytes;
  L.oob_w = wbytes;
  L.rx = make_rsrc(a.x, xbytes);
  L.rw = make_rsrc(a.w, wbytes);
  L.gelu = a.epilogue == G4_LINEAR_GELU_MUL;
  L.half = a.n / 2;

  constexpr int CB = T::CB;
  floatx4 acc[4][CB];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < CB; ++c) acc[r][c] = floatx4{0.f, 0.f, 0.f, 0.f};

  gemm_dma<TR>(b0, L.rx, L.rw, L.K, L.kbeg, true, xbytes, wbytes, L.w, L.lane, L.m0, L.gelu, L.half, L.tile);
  gemm_dma<TR>(b1, L.rx, L.rw, L.K, L.kbeg + kGemmKT, L.nst > 1, xbytes, wbytes, L.w, L.lane, L.m0, L.gelu, L.half,
               L.tile);
  gemm_dma<TR>(b2, L.rx, L.rw, L.K, L.kbeg + 2 * kGemmKT, L.nst > 2, xbytes, wbytes, L.w, L.lane, L.m0, L.gelu,
               L.half, L.tile);
  for (int s = 0; s < L.nst; s += 4) {
    gemm_step<TR>(b0, b3, acc, L, s);
    if (s + 1 < L.nst) gemm_step<TR>(b1, b0, acc, L, s + 1);
    if (s + 2 < L.nst) gemm_step<TR>(b2, b1, acc, L, s + 2);
    if (s + 3 < L.nst) gemm_step<TR>(b3, b2, acc, L, s + 3);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the trailing (zero) DMAs

  // lane (grp, col) holds Y[m = m0 + 64 wr + 16 rb + col][n = n0 + WCOLS wc + 16 cb + 4 grp + j]
  if (L.gelu) {  // cb < CB / 2: gate columns; cb + CB / 2: the up columns of the same outputs
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int m = L.m0 + 64 * L.wr + 16 * rb + L.col;
      if (m < a.m) {
#pragma unroll
        for (int cb = 0; cb < CB / 2; ++cb) {
          float y[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            y[j] = gelu_tanh_mul(round_bf16(acc[rb][cb][j]), round_bf16(acc[rb][cb + CB / 2][j]));
          uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + (int64_t)m * a.ldy + L.tile * (T::TC / 2) +
                          (T::WCOLS / 2) * L.wc + 16 * cb + 4 * L.grp;
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int m = L.m0 + 64 * L.wr + 16 * rb + L.col;
    if (m < a.m) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int n = n0 + T::WCOLS * L.wc + 16 * cb + 4 * L.grp;
        if (a.ksplit == 1) {
          uint16_t* y = reinterpret_cast<uint16_t*>(a.y) + (int64_t)m * a.ldy + n;
          *reinterpret_cast<uint2*>(y) = make_uint2(pack_bf16x2(acc[rb][cb][0], acc[rb][cb][1]),
                                                    pack_bf16x2(acc[rb][cb][2], acc[rb][cb][3]));
        } else {
          float* p = partials + ((int64_t)split * a.m + m) * a.n + n;
          *reinterpret_cast<floatx4*>(p) = acc[rb][cb];
        }
      }
    }
  }
}

// Y = sum of the split partials (split order), rounded to bf16; 4 outputs per thread.
__global__ __launch_bounds__(256) void linear_reduce_kernel(G4LinearArgs a, const float* partials) {
  const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t total = (int64_t)a.m * a.n;
  if (i4 >= total) return;
  floatx4 s = *reinterpret_cast<const floatx4*>(partials + i4);
  for (int k = 1; k < a.ksplit; ++k) s += *reinterpret_cast<const floatx4*>(partials + (int64_t)k * total + i4);
  const int64_t m = i4 / a.n, n = i4 - m * a.n;
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y) + m * a.ldy + n;
  *reinterpret_cast<uint2*>(y) = make_uint2(pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]));
}

}  // namespace
}  // namespace g4

extern "C" size_t g4_linear_workspace_size(const G4LinearArgs* args) {
  if (!args || args->ksplit <= 1 || args->m <= 0 || args->n <= 0) return 0;
  return (size_t)args->ksplit * (size_t)args->m * (size_t)args->n * 4u;
}

extern "C" int g4_linear_bf16(const G4LinearArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_linear_bf16: args is NULL");
  const G4LinearArgs& a = *args;
  if (!a.x || !a.w || (!a.y && a.ksplit <= 1)) return fail(G4_ERR_INVALID, "g4_linear_bf16: NULL x/w/y");
  if (a.m <= 0 || a.m > kGemmRows) return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: m %d (1..%d)", a.m, kGemmRows);
  if (a.n <= 0 || a.n % 64) return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: n %d (a multiple of 64)", a.n);
  if (a.ksplit < 1 || a.ksplit > 64) return fail(G4_ERR_INVALID, "g4_linear_bf16: ksplit %d (1..64)", a.ksplit);
  if (a.k <= 0 || a.k % (kGemmKT * a.ksplit))
    return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: k %d (a multiple of %d x ksplit %d)", a.k, kGemmKT, a.ksplit);
  if ((int64_t)a.m * a.k * 2 >= (int64_t)1 << 31 || (int64_t)a.n * a.k * 2 >= (int64_t)1 << 31)
    return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: operands beyond 2 GiB");
  if (a.epilogue != G4_LINEAR_PLAIN && a.epilogue != G4_LINEAR_GELU_MUL)
    return fail(G4_ERR_INVALID, "g4_linear_bf16: epilogue %d", a.epilogue);
  if (a.epilogue == G4_LINEAR_GELU_MUL && (a.ksplit != 1 || !a.y))
    return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: the gated-GELU epilogue needs ksplit 1 and y");
  const int ycols = a.epilogue == G4_LINEAR_GELU_MUL ? a.n / 2 : a.n;
  if (a.y && (a.ldy < ycols || a.ldy % 4))
    return fail(G4_ERR_INVALID, "g4_linear_bf16: ldy %d (>= n, a multiple of 4)", a.ldy);
  if ((reinterpret_cast<uintptr_t>(a.y) & 7) || (reinterpret_cast<uintptr_t>(a.x) & 15) ||
      (reinterpret_cast<uintptr_t>(a.w) & 15))
    return fail(G4_ERR_INVALID, "g4_linear_bf16: x/w need 16-byte and y 8-byte alignment");
  const size_t need = g4_linear_workspace_size(args);
  if (need && (!a.workspace || a.workspace_bytes < need))
    return fail(G4_ERR_WORKSPACE, "g4_linear_bf16: ksplit %d needs %zu B of workspace (have %zu)", a.ksplit, need,
                a.workspace ? a.workspace_bytes : (size_t)0);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* partials = reinterpret_cast<float*>(a.workspace);
  // 128 x 128 tiles when the rows fill two halves and the columns divide by 128; else 256 x 64
  if (a.m > 128 && a.n % 128 == 0)
    hipLaunchKernelGGL(linear_bf16_kernel<128>, dim3((unsigned)(a.n / 128 * a.ksplit * 2)), dim3(GemmTile<128>::THREADS), 0,
                       st, a, partials);
  else
    hipLaunchKernelGGL(linear_bf16_kernel<256>, dim3((unsigned)(a.n / 64 * a.ksplit)), dim3(GemmTile<256>::THREADS), 0, st,
                       a, partials);
  if (int rc = check_launch("g4_linear_bf16")) return rc;
  if (a.ksplit > 1 && a.y) {  // without y the partials stay in the workspace for the consumer
    const int64_t quads = ((int64_t)a.m * a.n) / 4;
    hipLaunchKernelGGL(linear_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, a,
                       (const float*)partials);
    return check_launch("g4_linear_bf16 (split-K sum)");
  }
  return G4_OK;
}
