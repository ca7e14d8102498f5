// resident_k2.hip — the resident decode kernel for up to 2 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic; with the barrier
// exchange and with the polling exchange.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_2(int dh, bool poll) {
  if (poll) return dh == 64 ? (const void*)k_resident<2, 64, true> : (const void*)k_resident<2, 0, true>;
  return dh == 64 ? (const void*)k_resident<2, 64> : (const void*)k_resident<2, 0>;
}

}  // namespace mitok
