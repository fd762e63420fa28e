// Library-level entry points of libllmy that are not tied to one kernel.
#include "abi_util.hpp"

extern "C" int32_t llmy_abi_version(void) { return 1; }
