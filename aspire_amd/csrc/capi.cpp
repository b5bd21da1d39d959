// Error state and build identity of libaspire_hip.
#include "common.h"

#ifndef ASPIRE_BUILD_FLAGS
#define ASPIRE_BUILD_FLAGS "unknown"
#endif
#ifndef ASPIRE_SOURCE_SHA256
#define ASPIRE_SOURCE_SHA256 "unknown"
#endif

namespace aspire {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

const char* last_error() { return g_last_error.c_str(); }

}  // namespace aspire

extern "C" const char* aspire_last_error(void) { return aspire::last_error(); }

#define ASPIRE_STR2(x) #x
#define ASPIRE_STR(x) ASPIRE_STR2(x)

extern "C" const char* aspire_build_info(void) {
  return "libaspire_hip 0.1 target=gfx950 hip=" ASPIRE_STR(HIP_VERSION_MAJOR) "." ASPIRE_STR(
      HIP_VERSION_MINOR) "." ASPIRE_STR(HIP_VERSION_PATCH) " sources_sha256=" ASPIRE_SOURCE_SHA256
                                                           " flags=" ASPIRE_BUILD_FLAGS;
}

extern "C" int32_t aspire_max_kv_tile(void) { return aspire::kPage; }
