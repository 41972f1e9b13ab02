// Device-type -> runtime function table (reference: src/device/runtime_api.cpp:73-88).
#pragma once

#include "llaisys/runtime.h"

namespace llaisys::device {
const LlaisysRuntimeAPI *getRuntimeAPI(llaisysDeviceType_t type);
const LlaisysRuntimeAPI *cpuRuntimeAPI();
const LlaisysRuntimeAPI *hipRuntimeAPI();
const LlaisysRuntimeAPI *unsupportedRuntimeAPI();
} // namespace llaisys::device
