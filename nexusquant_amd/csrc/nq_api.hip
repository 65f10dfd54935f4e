// Host-side error plumbing and version query of the C ABI.
#include <stdarg.h>

#include "nq_common.h"

namespace nq {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

}  // namespace nq

#ifndef NQ_SOURCE_HASH
#error "build with -DNQ_SOURCE_HASH=<hash of the sources> (python -m nexusquant_amd.build)"
#endif

extern "C" int nq_abi_version(void) { return NQ_ABI_VERSION; }

extern "C" const char* nq_source_hash(void) { return NQ_SOURCE_HASH; }

extern "C" const char* nq_last_error(void) { return nq::g_last_error; }
