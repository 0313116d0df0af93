// The float64 SSD chunk scan (ssd64.hip): the entry points of mko_ssd_* for x_dtype MKO_F64.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "../../include/mko.h"

namespace mko {

size_t ssd64_saved_bytes(const mko_ssd_params* prm);
size_t ssd64_bwd_workspace_size(const mko_ssd_params* prm);
int ssd64_fwd(const mko_ssd_params* prm, hipStream_t s);
int ssd64_bwd(const mko_ssd_params* prm, hipStream_t s);

}  // namespace mko
