// Stand-in for <hip/hip_runtime.h> when the library's kernel sources are compiled for
// the CPU executor in tests/cpu_emu (test infrastructure, never shipped): the HIP
// keywords, vector types, runtime calls and gfx950 builtins the sources use, mapped
// onto the executor in ../../emu.h.
#pragma once
#include "../../emu.h"
