// Thread-local error state behind mpq_last_error() / mpq_last_error_code().
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace mpq {

static thread_local char g_error[1024] = {0};
static thread_local int g_error_code = 0;

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_error; }
int last_error_code() { return g_error_code; }
void set_error_code(int code) { g_error_code = code; }

}  // namespace mpq

extern "C" const char* mpq_last_error(void) { return mpq::last_error(); }
extern "C" int mpq_last_error_code(void) { return mpq::last_error_code(); }
extern "C" void mpq_clear_error(void) {
  mpq::set_error("%s", "");
  mpq::set_error_code(0);
}
