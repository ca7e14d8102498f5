// resident_k8.hip — the resident decode kernel for up to 8 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_8(int dh) {
  return dh == 64 ? (const void*)k_resident<8, 64> : (const void*)k_resident<8, 0>;
}

}  // namespace mitok
