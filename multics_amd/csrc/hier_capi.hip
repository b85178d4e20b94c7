// Library-wide C entry points: error string and version.
#include "hier_common.h"

namespace hier {
thread_local char g_last_error[512] = {0};
}

extern "C" const char* hier_last_error(void) { return hier::g_last_error; }

extern "C" const char* hier_version(void) { return "hierattn 0.1 gfx950"; }
