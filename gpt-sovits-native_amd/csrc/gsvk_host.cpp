// gsvk_host.cpp — host-only parts of the C ABI: version, status text, launch-status check and the
// sinusoidal PE table builder (init-time work, run once per model on the host like the reference).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>

#include "gsvk.h"

namespace gsvk {

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GSVK_OK : GSVK_E_HIP;
}

}  // namespace gsvk

extern "C" const char* gsvk_version(void) { return "gsvk 0.1.0 (gfx950)"; }

extern "C" const char* gsvk_status_string(int status) {
  switch (status) {
    case GSVK_OK: return "ok";
    case GSVK_E_NULL: return "required pointer is NULL";
    case GSVK_E_SIZE: return "zero or out-of-range size";
    case GSVK_E_DTYPE: return "unknown dtype, index type or activation";
    case GSVK_E_ALIAS: return "output overlaps an input";
    case GSVK_E_ARG: return "invalid argument";
    case GSVK_E_HIP: return "HIP launch error";
    case GSVK_E_FORMAT: return "malformed .gsv container";
    case GSVK_E_IO: return "cannot open or map the file";
    default: return "unknown status";
  }
}

// T2SEngine::pe_row (t2s_engine.cpp:711-720) for one position. The steps are kept as the
// reference writes them because the table values define the bit-exact gather output: a float log
// increment, float exp of float(d)*log_inc, and float sin/cos of float(pos)*div.
static void pe_row_into(float* row, size_t pos, size_t D) {
  const float log_inc = static_cast<float>(-std::log(10000.0) / static_cast<double>(D));
  const float p = static_cast<float>(pos);
  for (size_t d = 0; d < D; d += 2) {
    const float div = std::exp(static_cast<float>(d) * log_inc);
    const float ang = p * div;
    row[d] = std::sin(ang);
    row[d + 1] = std::cos(ang);
  }
}

extern "C" int gsvk_pe_table(float* host_out, size_t max_pos, size_t D) {
  if (!host_out) return GSVK_E_NULL;
  if (max_pos == 0 || D == 0 || max_pos > (1ul << 32) || D > (1ul << 24)) return GSVK_E_SIZE;
  if (D % 2) return GSVK_E_ARG;
  for (size_t pos = 0; pos < max_pos; ++pos) pe_row_into(host_out + pos * D, pos, D);
  return GSVK_OK;
}

extern "C" int gsvk_pe_row(float* host_out, size_t pos, size_t D) {
  if (!host_out) return GSVK_E_NULL;
  if (D == 0 || D > (1ul << 24) || pos > (1ul << 32)) return GSVK_E_SIZE;
  if (D % 2) return GSVK_E_ARG;
  pe_row_into(host_out, pos, D);
  return GSVK_OK;
}
