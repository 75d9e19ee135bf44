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
int local_step(const sfx_params& p, const sfx_batch& bt, bool global_on,
               int32_t* draft, int32_t* num_valid, int32_t* new_counts,
               const StepWs& ws, hipStream_t stream);

int check_global(const sfx_params& p, const sfx_index& ix);
int global_step(const sfx_params& p, const sfx_index& ix,
                const sfx_batch& bt, int32_t* draft, int32_t* num_valid,
                const StepWs& ws, hipStream_t stream);

}  // namespace sfx
