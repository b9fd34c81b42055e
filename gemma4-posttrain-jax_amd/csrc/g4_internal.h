// Host-side helpers shared by the C-ABI launchers: thread-local error text and argument checks.
#pragma once

#include <stdint.h>

#include "../../include/g4_rollout.h"

namespace g4 {

// Records a formatted message for g4_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a hipError_t of the launch just made to G4_OK / G4_ERR_LAUNCH.
int check_launch(const char* what);

// Devices the per-device set-up tracks (device ordinals 0 .. kMaxDevices - 1).
constexpr int kMaxDevices = 64;

// The library's one-time set-up of the current device (g4_init): raises the dynamic-LDS limit of
// every kernel that launches with more than the 64 KiB default. Runs once per device (std::call_once,
// so concurrent first calls wait for one set-up); later calls only read the recorded result.
// Returns G4_OK or the set-up's error code (message via g4_last_error), and the device ordinal.
int device_setup(int* device);

// Per-source set-up steps run by device_setup for `device` (the current device). A step records
// what it could not set up per kernel (see raise_lds_limit) and fails only on errors that leave no
// path of its source usable.
int setup_decode_kernels(int device);
int setup_prefill_kernels(int device);
int setup_lm_head(int device);

// Raises kernel `fn`'s dynamic-LDS limit to `bytes` on `device` (the current device; called from the
// set-up steps only) and records whether that worked. lds_limit_raised(device, fn) reads the record
// after device_setup: a launcher whose kernel needs the raised limit checks it, so a kernel whose
// limit could not be raised disables only the paths that launch it.
bool raise_lds_limit(int device, const void* fn, int bytes);
bool lds_limit_raised(int device, const void* fn);

// Head dims with an instantiated kernel: powers of two 8..512 (bf16 attention: 32..256).
inline bool supported_head_dim(int d) { return d >= 8 && d <= 512 && (d & (d - 1)) == 0; }

}  // namespace g4
