// General speculative acceptance ("Mode F") on gfx950 — see capi_general.cpp.
#include "common.h"
