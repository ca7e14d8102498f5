// resident_k4.hip — the resident decode kernel for up to 4 sequence(s)
// (resident.hpp); head dim 64 specialised, others generic; with the barrier
// exchange and with the polling exchange.
#include "resident.hpp"

namespace mitok {

const void* resident_kernel_4(int dh, bool poll) {
  if (poll) return dh == 64 ? (const void*)k_resident<4, 64, true> : (const void*)k_resident<4, 0, true>;
  return dh == 64 ? (const void*)k_resident<4, 64> : (const void*)k_resident<4, 0>;
}

}  // namespace mitok
