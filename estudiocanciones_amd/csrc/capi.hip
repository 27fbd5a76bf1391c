// Library-level entry points.
#include "common.h"

extern "C" const char* ecd_version(void) { return "ecdecode 0.1 gfx950"; }
