// Host-only entry points of libg4rollout.so: error reporting, version, and the integer
// metadata functions (KV-sharing map, ring-slot positions) that need no device.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "g4_common.h"
#include "g4_internal.h"

namespace g4 {

static thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(G4_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return G4_OK;
}

namespace {

std::once_flag g_setup_once[kMaxDevices];
int g_setup_status[kMaxDevices];
char g_setup_error[kMaxDevices][512];

// Kernels whose dynamic-LDS limit the set-up raised, per device (written under the device's
// std::call_once, read after it).
constexpr int kMaxLdsKernels = 64;
struct LdsRecord {
  const void* fn;
  bool ok;
};
LdsRecord g_lds[kMaxDevices][kMaxLdsKernels];
int g_lds_count[kMaxDevices];

}  // namespace

bool raise_lds_limit(int device, const void* fn, int bytes) {
  const bool ok = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
  if (!ok) (void)hipGetLastError();  // the failure is recorded here, not left for the next launch to report
  if (g_lds_count[device] < kMaxLdsKernels) g_lds[device][g_lds_count[device]++] = LdsRecord{fn, ok};
  return ok;
}

bool lds_limit_raised(int device, const void* fn) {
  for (int i = 0; i < g_lds_count[device]; ++i)
    if (g_lds[device][i].fn == fn) return g_lds[device][i].ok;
  return false;
}

int device_setup(int* device) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(G4_ERR_LAUNCH, "g4_init: no current HIP device (or ordinal %d >= %d)", dev, kMaxDevices);
  std::call_once(g_setup_once[dev], [dev] {
    int rc = setup_decode_kernels(dev);
    if (rc == G4_OK) rc = setup_prefill_kernels(dev);
    if (rc == G4_OK) rc = setup_lm_head(dev);
    if (rc != G4_OK) snprintf(g_setup_error[dev], sizeof(g_setup_error[dev]), "%s", g_error);
    g_setup_status[dev] = rc;
  });
  if (device) *device = dev;
  if (g_setup_status[dev] != G4_OK) return fail(g_setup_status[dev], "%s", g_setup_error[dev]);
  return G4_OK;
}

}  // namespace g4

extern "C" {

int g4_init(void) { return g4::device_setup(nullptr); }

const char* g4_last_error(void) { return g4::g_error; }

const char* g4_version(void) { return "g4rollout 0.1 (gfx950)"; }

// model.py:153-168: a layer i >= L - num_kv_shared reuses the K/V of the last non-shared layer
// of its own type; every other layer is its own source.
int g4_kv_source_layers(int32_t num_layers, int32_t num_kv_shared_layers, const int32_t* layer_types,
                        int32_t* out) {
  if (num_layers <= 0 || num_kv_shared_layers < 0 || num_kv_shared_layers > num_layers || !layer_types || !out)
    return g4::fail(G4_ERR_INVALID, "g4_kv_source_layers: invalid arguments");
  const int32_t first_shared = num_layers - num_kv_shared_layers;
  for (int32_t i = 0; i < num_layers; ++i) {
    if (layer_types[i] != 0 && layer_types[i] != 1)
      return g4::fail(G4_ERR_INVALID, "g4_kv_source_layers: layer_types[%d]=%d is not 0/1", i, layer_types[i]);
    if (num_kv_shared_layers == 0 || i < first_shared) {
      out[i] = i;
      continue;
    }
    int32_t src = -1;
    for (int32_t j = first_shared - 1; j >= 0; --j) {
      if (layer_types[j] == layer_types[i]) {
        src = j;
        break;
      }
    }
    if (src < 0)
      return g4::fail(G4_ERR_INVALID, "g4_kv_source_layers: no non-shared layer of the type of layer %d", i);
    out[i] = src;
  }
  return G4_OK;
}

int g4_ring_slot_positions(int32_t last_written, int32_t window_capacity, int32_t* out) {
  if (window_capacity <= 0 || !out) return g4::fail(G4_ERR_INVALID, "g4_ring_slot_positions: invalid arguments");
  for (int32_t r = 0; r < window_capacity; ++r)
    out[r] = (int32_t)g4::ring_slot_position(last_written, r, window_capacity);
  return G4_OK;
}

}  // extern "C"
