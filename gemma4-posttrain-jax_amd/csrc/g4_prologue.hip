// One decode step's input glue in one launch (g4_decode_prologue): the embedding gather and
// scale (model.py:599-600), the key-mask update at the write slot (model.py:608-610) and the
// rotary tables of the step's positions for each layer type (model.py:288-306, 624-627).
// One workgroup per batch row. Rounding as the reference: x = bf16(f32(embed[token]) * scale),
// freqs = f32(position) * inv_freq in f32, cos / sin in f32 of concat(freqs, freqs).
#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kPrologueThreads = 256;

__global__ __launch_bounds__(kPrologueThreads) void decode_prologue_kernel(G4PrologueArgs a) {
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  int tok = a.tokens[b];
  tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);  // an id outside the table reads its edge row
  const uint16_t* erow = reinterpret_cast<const uint16_t*>(a.embed) + (int64_t)tok * a.hidden;
  uint16_t* xrow = reinterpret_cast<uint16_t*>(a.x_out) + (int64_t)b * a.hidden;
  for (int g = t; g < a.hidden / 8; g += kPrologueThreads) {
    float v[8];
    unpack8(load16(erow + 8 * g), v);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= a.embed_scale;
    *reinterpret_cast<u32x4*>(xrow + 8 * g) = pack8(v);
  }
  const float pos = (float)a.positions[b];
  for (int i = 0; i < a.n_tables; ++i) {
    const int D = a.rot_dim[i], half = D / 2;
    for (int d = t; d < D; d += kPrologueThreads) {
      const float f = pos * a.inv_freq[i][d < half ? d : d - half];
      a.cos_out[i][(int64_t)b * D + d] = cosf(f);
      a.sin_out[i][(int64_t)b * D + d] = sinf(f);
    }
  }
  if (t == 0) {
    const int s = a.slot[b];
    if (s >= 0 && s < a.key_mask_stride) a.key_mask[(int64_t)b * a.key_mask_stride + s] = a.active[b] ? 1 : 0;
  }
}

}  // namespace
}  // namespace g4

extern "C" int g4_decode_prologue(const G4PrologueArgs* args, void* stream) {
  using namespace g4;
  if (!args) return fail(G4_ERR_INVALID, "g4_decode_prologue: args is NULL");
  const G4PrologueArgs& a = *args;
  if (a.batch <= 0 || a.hidden <= 0 || a.hidden % 8 || a.vocab <= 0)
    return fail(G4_ERR_INVALID, "g4_decode_prologue: batch %d hidden %d (a multiple of 8) vocab %d", a.batch,
                a.hidden, a.vocab);
  if (!a.tokens || !a.positions || !a.active || !a.slot || !a.key_mask || !a.embed || !a.x_out)
    return fail(G4_ERR_INVALID, "g4_decode_prologue: NULL pointer");
  if (a.key_mask_stride <= 0) return fail(G4_ERR_INVALID, "g4_decode_prologue: key_mask_stride %d", a.key_mask_stride);
  if ((reinterpret_cast<uintptr_t>(a.embed) | reinterpret_cast<uintptr_t>(a.x_out)) & 15)
    return fail(G4_ERR_INVALID, "g4_decode_prologue: embed and x_out need 16-byte alignment");
  if (a.n_tables < 0 || a.n_tables > 2) return fail(G4_ERR_INVALID, "g4_decode_prologue: n_tables %d", a.n_tables);
  for (int i = 0; i < a.n_tables; ++i)
    if (a.rot_dim[i] <= 0 || a.rot_dim[i] % 2 || !a.inv_freq[i] || !a.cos_out[i] || !a.sin_out[i])
      return fail(G4_ERR_INVALID, "g4_decode_prologue: rotary table %d (dim %d)", i, a.rot_dim[i]);
  hipLaunchKernelGGL(decode_prologue_kernel, dim3(a.batch), dim3(kPrologueThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("g4_decode_prologue");
}
