// Library identification.
#include "common.h"

#ifndef MLCG_BUILD_ID
#define MLCG_BUILD_ID "dev"
#endif

extern "C" const char* mlcg_version(void) { return "libmlcg_hip " MLCG_BUILD_ID " gfx950"; }
