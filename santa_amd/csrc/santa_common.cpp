// santa_common.cpp -- error reporting and version of the C ABI.
#include <cstdarg>
#include <cstdio>

#include "santa_amd.h"
#include "santa_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace santa {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_last_error[0] = '\0';
  return SANTA_OK;
}

int check_page_table(const int* table, int num_pages, int page_size, int table_stride, int max_len, PageTable* pt) {
  if (!table) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  if (page_size < 8 || page_size > (1 << 20) || (page_size & (page_size - 1)) != 0)
    return set_error(SANTA_ERR_INVALID, "page_size must be a power of two in [8, 1048576]. Got page_size=%d", page_size);
  if (num_pages <= 0) return set_error(SANTA_ERR_INVALID, "num_pages must be > 0; got %d", num_pages);
  const long long need = (static_cast<long long>(max_len) + page_size - 1) / page_size;
  if (table_stride < need)
    return set_error(SANTA_ERR_INVALID, "block table too narrow: %d entries per sequence, %lld needed for %d tokens",
                     table_stride, need, max_len);
  int shift = 0;
  while ((1 << shift) < page_size) ++shift;
  *pt = PageTable{table, table_stride, shift, num_pages};
  return SANTA_OK;
}

}  // namespace santa

extern "C" const char* santa_last_error(void) { return g_last_error; }

extern "C" const char* santa_version(void) { return "santa_amd 0.1.0 (gfx950)"; }
