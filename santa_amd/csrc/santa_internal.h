// santa_internal.h -- host-side helpers shared by the C-ABI translation units.
#pragma once

#include <stddef.h>

namespace santa {

// Records a printf-style message as the calling thread's last error and
// returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error and returns SANTA_OK.
int clear_error();

constexpr size_t kWsAlign = 256;
inline size_t align_up(size_t x) { return (x + kWsAlign - 1) & ~(kWsAlign - 1); }

}  // namespace santa
