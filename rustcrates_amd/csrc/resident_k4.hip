// resident_k4.hip — the resident decode kernel for up to 4 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_4(int dh) {
  return dh == 64 ? (const void*)k_resident<4, 64> : (const void*)k_resident<4, 0>;
}

}  // namespace mitok
