// Contract verification and lowering of a sealed tb.pipeline_mainline onto
// the gfx950 launch configuration of include/tb_gfx950.h.
#pragma once

#include "plans.h"
#include "tb_gfx950.h"

namespace tb {

void verifyMainlineContract(const Module &m, const Op &mainline,
                            const KernelContract &k);
tb_gemm_config lowerContractToConfig(const KernelContract &k);

} // namespace tb
