// Decode-step projection GEMM (g4_linear_bf16): Y[M, N] = X[M, K] . W[N, K]^T, bf16 in, f32
// accumulation, bf16 out, for the rollout's decode batch (M <= 256 rows). Replaces the dense
// projections of forward_attention / forward_mlp (model.py:463-482, 393-396, 500) at S = 1.
//
// At M = 256 the projection is a stream of the weight matrix: every weight byte is used by all
// 256 rows once. One workgroup owns all M rows and 64 columns of W, so W is read from HBM exactly
// once, and X (shared by every workgroup) comes from L2. K is walked in stages of 64: the X
// stage (256 x 64) and the W stage (64 x 64) are DMA'd into a 4-deep LDS ring
// (buffer_load ... lds), three stages in flight while the fourth is multiplied.
//
// LDS layout of a stage: groups of 8 rows x 128 bytes (one DMA instruction: 64 lanes x 16 bytes,
// 8 full 128-byte lines of the row-major operand); within a group, row r's
// 16-byte piece kc sits at slot kc ^ r, so the 16 rows an MFMA operand read touches fall on
// different banks. Each lane DMAs the piece that belongs at its slot.
//
// MFMA v_mfma_f32_16x16x32_bf16 with A = 16 rows of W (output columns) and B = 16 rows of X
// (output rows): lane (grp, col) accumulates Y[m = 16 rb + col][n = 16 cb + 4 grp .. + 3], four
// consecutive outputs of one row. Wave w owns rows [64 w, 64 w + 64) x the workgroup's 64 columns
// (4 x 4 accumulator blocks).
//
// Split-K (ksplit > 1): workgroup (n-tile, s) covers K range s; partial sums go to an f32
// workspace [ksplit][M][N] and a second kernel adds them in split order and rounds to bf16, or,
// with no y given, they are left there for a consumer that adds them itself
// (g4_residual_norm_splitk, the residual norm after the MLP's down projection).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kGemmRows = 256;  // M rows per workgroup (all of them)
constexpr int kGemmCols = 64;   // N columns per workgroup
constexpr int kGemmKT = 64;     // K per stage
constexpr int kGemmThreads = 256;
constexpr int kGroupBytes = 1024;                   // 8 rows x 128 B (a 4-stage ring fills the 160 KiB)
constexpr int kXGroups = kGemmRows / 8;             // 32
constexpr int kWGroups = kGemmCols / 8;             // 8
constexpr int kStageBytes = (kXGroups + kWGroups) * kGroupBytes;
constexpr int kDmaPerWave = (kXGroups + kWGroups) / (kGemmThreads / 64);  // 10 DMA instructions per wave and stage

typedef unsigned char StageBuf[kStageBytes];

// DMA of stage `st` (K offset k0) into `buf`: wave w moves groups w, w + 4, ... of X then of W.
// Lane l of a group instruction takes row 8 g + l / 8 and the 16-byte piece (l % 8) ^ (row % 8) of
// its 128-byte K slice. W group j (rows 8 j .. 8 j + 7 of the tile) starts at weight row
// wrow[j >> 2] + 8 (j & 3). Past the last stage every load reads beyond its resource (zeros, no
// memory request), so every wave always issues kDmaPerWave loads per stage.
__device__ __forceinline__ void gemm_dma(unsigned char* __restrict__ buf, __amdgpu_buffer_rsrc_t rx,
                                         __amdgpu_buffer_rsrc_t rw, int K, int k0, bool live, uint32_t oob_x,
                                         uint32_t oob_w, int w, int lane, int wrow0, int wrow1) {
  const int rl = lane >> 3;                       // row within the group
  const int kc = (lane & 7) ^ rl;                 // 16-byte piece this lane fetches (row % 8 == rl)
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    const int g = w + 4 * i;  // groups 0..31: X, 32..39: W
    const bool is_x = g < kXGroups;
    const int gw = g - kXGroups;
    const int row = is_x ? 8 * g + rl : (gw < 4 ? wrow0 : wrow1) + 8 * (gw & 3) + rl;
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

__device__ __forceinline__ void gemm_compute(const unsigned char* __restrict__ buf, floatx4 (&acc)[4][4], int w,
                                             int col, int grp) {
  const uint32_t xs = lds_addr(buf);
  const uint32_t ws = xs + kXGroups * kGroupBytes;
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    u32x4 a[4], b[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) a[cb] = lds_read16(gemm_operand_at(ws, 16 * cb + col, 4 * kh + grp));
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) b[rb] = lds_read16(gemm_operand_at(xs, 64 * w + 16 * rb + col, 4 * kh + grp));
    __asm__ volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma16x16x32(as_bf16x8(a[cb]), as_bf16x8(b[rb]), acc[rb][cb]);
  }
}

// One pipeline step: stage s is in `cur`; `nxt` holds stage s + 1 (in flight, with s + 2); stage
// s + 3 is requested into `fre` (the buffer of stage s - 1, which every wave has finished with)
// after the stage's MFMAs are issued, so a DMA issue that waits for room in the memory queue
// does not hold them back (down projection 19.3 -> 18.6 us).
__device__ __forceinline__ void gemm_step(unsigned char* __restrict__ cur, unsigned char* __restrict__ nxt,
                                          unsigned char* __restrict__ fre, floatx4 (&acc)[4][4],
                                          __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw, int K, int kbeg,
                                          int s, int nst, uint32_t oob_x, uint32_t oob_w, int w, int lane, int col,
                                          int grp, int wrow0, int wrow1) {
  (void)nxt;
  // this wave's DMAs of stage s have landed (stages s + 1, s + 2 may not have), then every wave's
  __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * kDmaPerWave) : "memory");
  gemm_compute(cur, acc, w, col, grp);
  gemm_dma(fre, rx, rw, K, kbeg + (s + 3) * kGemmKT, s + 3 < nst, oob_x, oob_w, w, lane, wrow0, wrow1);
}

// grid: (N / 64) * ksplit workgroups, workgroup i = (column tile i / ksplit, K split i % ksplit).
// Workgroups are dealt to the 8 XCDs round robin (i mod 8), so with ksplit dividing 8 every XCD
// works on one K split and its L2 holds only that split's slice of X, which all its column tiles
// re-read. K / ksplit must be a multiple of 64. With the gated-GELU epilogue the workgroup's 64
// weight rows are 32 gate rows and the 32 up rows of the same output columns.
__global__ __launch_bounds__(kGemmThreads) void linear_bf16_kernel(G4LinearArgs a, float* partials) {
  __shared__ __attribute__((aligned(1024))) StageBuf b0, b1, b2, b3;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int tile = (int)blockIdx.x / a.ksplit;
  const int split = (int)blockIdx.x - tile * a.ksplit;
  const int n0 = tile * kGemmCols;
  const int K = a.k;
  const int kper = K / a.ksplit;
  const int kbeg = split * kper;
  const int nst = kper / kGemmKT;
  const uint32_t xbytes = (uint32_t)a.m * (uint32_t)K * 2u;  // rows >= M read as zeros
  const uint32_t wbytes = (uint32_t)a.n * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, xbytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, wbytes);
  const bool gelu = a.epilogue == G4_LINEAR_GELU_MUL;
  const int half = a.n / 2;
  // weight rows of tile groups 0..3 and 4..7
  const int wrow0 = gelu ? tile * 32 : n0;
  const int wrow1 = gelu ? half + tile * 32 : n0 + 32;

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  gemm_dma(b0, rx, rw, K, kbeg, true, xbytes, wbytes, w, lane, wrow0, wrow1);
  gemm_dma(b1, rx, rw, K, kbeg + kGemmKT, nst > 1, xbytes, wbytes, w, lane, wrow0, wrow1);
  gemm_dma(b2, rx, rw, K, kbeg + 2 * kGemmKT, nst > 2, xbytes, wbytes, w, lane, wrow0, wrow1);
  for (int s = 0; s < nst; s += 4) {
    gemm_step(b0, b1, b3, acc, rx, rw, K, kbeg, s, nst, xbytes, wbytes, w, lane, col, grp, wrow0, wrow1);
    if (s + 1 < nst)
      gemm_step(b1, b2, b0, acc, rx, rw, K, kbeg, s + 1, nst, xbytes, wbytes, w, lane, col, grp, wrow0, wrow1);
    if (s + 2 < nst)
      gemm_step(b2, b3, b1, acc, rx, rw, K, kbeg, s + 2, nst, xbytes, wbytes, w, lane, col, grp, wrow0, wrow1);
    if (s + 3 < nst)
      gemm_step(b3, b0, b2, acc, rx, rw, K, kbeg, s + 3, nst, xbytes, wbytes, w, lane, col, grp, wrow0, wrow1);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the trailing (zero) DMAs

  // lane (grp, col) holds Y[m = 64 w + 16 rb + col][n = n0 + 16 cb + 4 grp + j]
  if (gelu) {  // cb 0, 1: gate columns; cb 2, 3: the up columns of the same outputs
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int m = 64 * w + 16 * rb + col;
      if (m < a.m) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          float y[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) y[j] = gelu_tanh_mul(round_bf16(acc[rb][cb][j]), round_bf16(acc[rb][cb + 2][j]));
          uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + (int64_t)m * a.ldy + tile * 32 + 16 * cb + 4 * grp;
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int m = 64 * w + 16 * rb + col;
    if (m < a.m) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int n = n0 + 16 * cb + 4 * grp;
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
  if (a.n <= 0 || a.n % kGemmCols) return fail(G4_ERR_UNSUPPORTED, "g4_linear_bf16: n %d (a multiple of %d)", a.n, kGemmCols);
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
  hipLaunchKernelGGL(linear_bf16_kernel, dim3((unsigned)(a.n / kGemmCols * a.ksplit)), dim3(kGemmThreads), 0,
                     st, a, partials);
  if (int rc = check_launch("g4_linear_bf16")) return rc;
  if (a.ksplit > 1 && a.y) {  // without y the partials stay in the workspace for the consumer
    const int64_t quads = ((int64_t)a.m * a.n) / 4;
    hipLaunchKernelGGL(linear_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, a,
                       (const float*)partials);
    return check_launch("g4_linear_bf16 (split-K sum)");
  }
  return G4_OK;
}
