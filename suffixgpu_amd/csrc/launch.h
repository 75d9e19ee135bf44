// Host-side launchers shared between the translation units of the library.
#pragma once

#include <hip/hip_runtime.h>

#include "step_ws.h"
#include "suffixgpu_amd.h"

namespace sfx {

// LDS available to one workgroup on gfx950 (160 KiB per CU).
constexpr size_t kMaxLds = 160 * 1024;

int check_local(const sfx_params& p, const sfx_batch& bt);
size_t local_lds_bytes(const sfx_params& p, int64_t S);

int check_global(const sfx_params& p, const sfx_index& ix);
int mb_lds_bytes(const sfx_index& ix);
int merge_waves_for(const sfx_params& p, const sfx_index& ix, size_t* lds);

}  // namespace sfx
