// Helpers shared by the library's translation units (not part of the C ABI).
#pragma once

#include <stddef.h>

namespace z1detail {

// Dynamic LDS (bytes) that caps a launch at `per_cu` resident workgroups per CU on device `dev`; 0 when the
// device does not report its LDS size.  Returns Z1_OK or a hipError_t.
int occupancy_lds(int dev, int per_cu, size_t* bytes);

}  // namespace z1detail
