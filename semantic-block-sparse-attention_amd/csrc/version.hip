// ABI version of libsbsa.
#include "sbsa_common.h"

extern "C" int sbsa_abi_version(void) { return 4; }
