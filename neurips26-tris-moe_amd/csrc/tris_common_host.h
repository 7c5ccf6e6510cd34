// Host-only declarations shared by the C-ABI translation units.
#pragma once

#include "tris_moe_hip.h"

namespace tris {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace tris
