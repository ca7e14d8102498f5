// resident_k2.hip — the resident decode kernel for up to 2 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_2(int dh) {
  return dh == 64 ? (const void*)k_resident<2, 64> : (const void*)k_resident<2, 0>;
}

}  // namespace mitok
