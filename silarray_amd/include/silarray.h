#pragma once
// Umbrella header, as the reference's include/silarray.h:1-6.
#include "types.h"
#include "device.h"
#include "storage.h"
#include "gpu.h"
#include "array.h"
