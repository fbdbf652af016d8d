// Entry point of the MI355X HIP backend (libtraincpp_hip.so). A new sibling of
// the reference's cpu_device()/vulkan_device() (src/core/trc_backends.h:14-22):
// returns the Device of HIP ordinal `ordinal`, or nullptr when that GPU is not
// visible. Devices are process-lifetime singletons. The registry of this
// library (device_count/device_get) enumerates them automatically.
#pragma once

#include "trc_backend.h"

namespace traincpp {

Device* hip_device(int ordinal = 0);
int     hip_device_count();

}  // namespace traincpp
