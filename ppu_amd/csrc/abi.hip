// ABI version query; the value must match Q35_ABI_VERSION in include/q35.h.
#include "q35_common.hpp"

extern "C" int q35_abi_version(void) { return 1; }
