// Host-side helpers shared by the C-ABI launchers: thread-local error text and argument checks.
#pragma once

#include <stdint.h>

#include "../../include/g4_rollout.h"

namespace g4 {

// Records a formatted message for g4_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a hipError_t of the launch just made to G4_OK / G4_ERR_LAUNCH.
int check_launch(const char* what);

// Head dims with an instantiated kernel: powers of two 8..512 (bf16 attention: 32..256).
inline bool supported_head_dim(int d) { return d >= 8 && d <= 512 && (d & (d - 1)) == 0; }

}  // namespace g4
