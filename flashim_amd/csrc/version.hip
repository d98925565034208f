// Library version (the one entry point with no kernel behind it).
#include "common.h"

extern "C" int fim_version(void) { return 100; }
