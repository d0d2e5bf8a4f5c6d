// Internal helpers shared by the library's translation units (not part of the C ABI).
#ifndef PAGEDCORE_PC_INTERNAL_H
#define PAGEDCORE_PC_INTERNAL_H

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "pagedcore_hip.h"

namespace pc_internal {

// Records printf-style text for pc_last_error() on the calling thread; returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's error text; returns PC_OK.
int ok();

// PC_LAUNCH error naming `what` if the last kernel launch failed, else ok().
int check_launch(const char* what);

// The calling thread's error text.
const char* last_error();

inline bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace pc_internal

#endif  // PAGEDCORE_PC_INTERNAL_H
