// TEST INFRASTRUCTURE ONLY: see hip_runtime.h (the library declares no
// extension call that its host code makes).
#pragma once
#include "hip_runtime.h"
