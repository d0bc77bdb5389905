// Internal definition of the opaque tb_gemm_desc (include/tb_gfx950.h).
#pragma once

#include "tb_gfx950.h"

#include <cstddef>
#include <string>

namespace tbk {
struct KernelEntry;
}

struct tb_gemm_desc {
  tb_gemm_config cfg{};
  const tbk::KernelEntry *entry = nullptr;
  int out_mode = 0;
  int64_t tiles_m = 0, tiles_n = 0, tiles_k = 0;
  int64_t total_work = 0;
  int64_t lds_bytes = 0;
  size_t workspace_bytes = 0;
};

namespace tbrt {
// Validates a flattened config and binds it to a compiled kernel instance.
int create_desc(const tb_gemm_config &c, tb_gemm_desc **out);
// Sets the thread-local message returned by tb_last_error().
void set_error(const std::string &msg);
// The s_waitcnt depths compiled into the descriptor's kernel instance:
// {vmcnt at the prologue, vmcnt at the per-k-tile barrier, lgkmcnt there}.
void desc_waits(const tb_gemm_desc *d, int64_t out[3]);
} // namespace tbrt
