// resident_k8.hip — the resident decode kernel for up to 8 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic; with the barrier
// exchange and with the polling exchange.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_8(int dh, bool poll) {
  if (poll) return dh == 64 ? (const void*)k_resident<8, 64, true> : (const void*)k_resident<8, 0, true>;
  return dh == 64 ? (const void*)k_resident<8, 64> : (const void*)k_resident<8, 0>;
}

}  // namespace mitok
