// generate's per-step bookkeeping (g4_rollout_step, sampler.py:279-296): the masked token and
// log-probability of the step's draw into the completion arrays, the EOS update of the active rows
// and the next decode step's inputs, in one launch of one workgroup (one thread per row) instead
// of a dozen framework kernels.
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kRolloutThreads = 1024;
constexpr int kEosRowLoop = 64;  // up to this many EOS ids each row scans them; more: the ids are split over the threads

// One workgroup; rows in blocks of blockDim.x (thread t takes row b0 + t of each block). The EOS
// test of a row block: with few ids each row scans them (staged in LDS, 16-byte reads padded with a
// copy of the first id, which changes no match); with many, each thread holds up to four ids per
// pass and scans the block's tokens (LDS broadcast reads of four rows), flagging the rows that
// match, so a thread does rows x 4 compares per pass instead of one per id; such a launch takes
// 1024 threads whatever the batch (4096 ids at B = 256: one pass, ~150 us -> a few us per step).
__global__ __launch_bounds__(kRolloutThreads) void rollout_step_kernel(G4RolloutStepArgs a) {
  __shared__ __attribute__((aligned(16))) int32_t eos_lds[kEosRowLoop];
  __shared__ __attribute__((aligned(16))) int32_t tok_lds[kRolloutThreads];
  __shared__ int32_t hit_lds[kRolloutThreads];
  bool stays_any = false;
  const int nt = (int)blockDim.x;
  for (int b0 = 0; b0 < a.batch; b0 += nt) {
    const int b = b0 + (int)threadIdx.x;
    const bool row = b < a.batch;
    const bool act = row && a.active[b] != 0;           // the step's mask
    const int32_t tok = act ? a.sampled[b] : a.pad_id;  // finished rows emit pad
    bool eos = false;
    if (a.n_eos <= kEosRowLoop) {
      if (a.n_eos > 0) {
        const int n4 = (a.n_eos + 3) / 4 * 4;
        __syncthreads();  // the previous row block's readers are done
        for (int i = threadIdx.x; i < n4; i += nt) eos_lds[i] = a.eos_ids[i < a.n_eos ? i : 0];
        __syncthreads();
        const int4* ids4 = reinterpret_cast<const int4*>(eos_lds);
        for (int i = 0; i < n4 / 4; ++i) {
          const int4 e = ids4[i];
          eos = eos || tok == e.x || tok == e.y || tok == e.z || tok == e.w;
        }
      }
    } else {
      const int nrows = a.batch - b0 < nt ? a.batch - b0 : nt;
      __syncthreads();  // the previous row block's readers are done
      tok_lds[threadIdx.x] = tok;
      hit_lds[threadIdx.x] = 0;
      __syncthreads();
      for (int c0 = 0; c0 < a.n_eos; c0 += 4 * nt) {
        const int i0 = c0 + (int)threadIdx.x;
        if (i0 < a.n_eos) {  // ids i0, i0 + nt, ... of this pass (a missing one repeats the first)
          const int32_t e0 = a.eos_ids[i0];
          const int32_t e1 = i0 + nt < a.n_eos ? a.eos_ids[i0 + nt] : e0;
          const int32_t e2 = i0 + 2 * nt < a.n_eos ? a.eos_ids[i0 + 2 * nt] : e0;
          const int32_t e3 = i0 + 3 * nt < a.n_eos ? a.eos_ids[i0 + 3 * nt] : e0;
          const int4* t4 = reinterpret_cast<const int4*>(tok_lds);  // four rows per read
          for (int r4 = 0; r4 < (nrows + 3) / 4; ++r4) {
            const int4 t = t4[r4];
            const int32_t tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = 4 * r4 + q;
              if (r < nrows && (tv[q] == e0 || tv[q] == e1 || tv[q] == e2 || tv[q] == e3)) hit_lds[r] = 1;
            }
          }
        }
      }
      __syncthreads();
      eos = hit_lds[threadIdx.x] != 0;
    }
    if (!row) continue;
    const int64_t at = (int64_t)b * a.max_new + a.step;
    if (a.id_bytes == 8) reinterpret_cast<int64_t*>(a.completion_ids)[at] = tok;
    else reinterpret_cast<int32_t*>(a.completion_ids)[at] = tok;
    a.completion_mask[at] = act ? 1 : 0;
    a.rollout_logps[at] = act ? a.logp[b] : 0.f;
    const bool stays = act && !eos;
    stays_any = stays_any || stays;
    if (a.next_token) a.next_token[b] = tok;
    if (a.next_pos) a.next_pos[b] = a.prompt_lengths[b] + a.step;
    if (a.next_mask) a.next_mask[b] = act ? 1 : 0;
    a.active[b] = stays ? 1 : 0;
  }
  const int any = __syncthreads_or(stays_any ? 1 : 0);
  if (threadIdx.x == 0 && a.any_active) *a.any_active = any ? 1 : 0;
}

}  // namespace
}  // namespace g4

extern "C" int g4_rollout_step(const G4RolloutStepArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_rollout_step: args is NULL");
  const G4RolloutStepArgs& a = *args;
  if (a.batch <= 0) return fail(G4_ERR_INVALID, "g4_rollout_step: batch %d", a.batch);
  if (a.max_new <= 0 || a.step < 0 || a.step >= a.max_new)
    return fail(G4_ERR_INVALID, "g4_rollout_step: step %d outside [0, max_new = %d)", a.step, a.max_new);
  if (a.id_bytes != 4 && a.id_bytes != 8) return fail(G4_ERR_INVALID, "g4_rollout_step: id_bytes %d", a.id_bytes);
  if (a.n_eos < 0 || (a.n_eos > 0 && !a.eos_ids)) return fail(G4_ERR_INVALID, "g4_rollout_step: eos_ids / n_eos");
  if (!a.sampled || !a.logp || !a.active || !a.completion_ids || !a.completion_mask || !a.rollout_logps ||
      (a.next_pos && !a.prompt_lengths))
    return fail(G4_ERR_INVALID, "g4_rollout_step: NULL pointer");
  if (reinterpret_cast<uintptr_t>(a.completion_ids) % (uintptr_t)a.id_bytes)
    return fail(G4_ERR_INVALID, "g4_rollout_step: completion_ids not %d-byte aligned", a.id_bytes);
  // a large EOS set is split over the threads: take all of them whatever the batch
  const int threads = a.batch < kRolloutThreads && a.n_eos <= kEosRowLoop ? (a.batch + 63) / 64 * 64 : kRolloutThreads;
  hipLaunchKernelGGL(rollout_step_kernel, dim3(1), dim3(threads), 0, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("g4_rollout_step");
}
