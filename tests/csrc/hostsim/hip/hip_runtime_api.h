// TEST INFRASTRUCTURE ONLY: see hip_runtime.h.
#pragma once
#include "hip_runtime.h"
