// C-ABI plumbing shared by all entry points: thread-local error text and the
// library version.
#include <cstdarg>

#include "imi_common.hpp"

namespace imi {

static thread_local char g_error[1024] = {0};

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace imi

extern "C" const char* imi_last_error(void) { return imi::g_error; }

extern "C" int imi_version(void) { return 5; }
