// gemm_mfma.hip — the MFMA-tiled complex GEMM for products of more than 64
// rows (the prompt pass): multiply_complex (utils/matrix.rs:16-65) with the
// epilogues of epilogue.hpp and the fused greedy id.
//
// This file is compiled on its own with -mllvm -amdgpu-mfma-vgpr-form=1
// (rustcrates_amd/build.py).  By default the compiler kept the accumulators
// in AGPRs for the MFMAs but carried them across the K loop in VGPRs, so every
// K step copied all 64 of them back (64 v_accvgpr_write per step) and waited
// for the tile loads before the first MFMA.  In the VGPR form the loop has no
// copies.  Measured on MI355X at config 3, batch 32 (prompt pass GEMMs per
// generate call): 10.68 -> 10.04 ms, 67.6% -> 71.9% of the FP64 MFMA peak.
// The flag is kept to this file: the skinny decode products measured slower
// with it.
#include "epilogue.hpp"

namespace mitok {

// ===========================================================================
// MFMA complex GEMM.  Block tile 64x64 (4 waves of 32x32), K step 16, operands
// de-interleaved into re/im planes in LDS (double-buffered).  Per 16x16x4 step
// a wave issues 4 v_mfma_f64_16x16x4_f64 per output tile:
//     Cr += Ar*Br;  Cr += (-Ai)*Bi;  Ci += Ar*Bi;  Ci += Ai*Br
// Lane layout of v_mfma_f64_16x16x4_f64 (wave64): A[i][k] at lane i+16k,
// B[k][j] at lane j+16k, D[i][j] at lane j+16*(i%4), element i/4 (unlike the
// f32 16x16x4 form, consecutive output rows sit in consecutive lane groups).
// blockIdx.z splits K; the last block of a tile sums the partials.
// ===========================================================================
constexpr int GPAD = 4;  // LDS row padding (doubles)

// MODE: the epilogue mode, fixed at compile time so each launch carries only
// its own epilogue (the GELU code is not inlined into the other products).
template <int MODE>
__global__ __launch_bounds__(256) void k_zgemm_mfma(const double2* __restrict__ A, long lda,
                                                       const double2* __restrict__ Bm, long ldb, int M, int N, int K,
                                                       int kchunk, Epi ep_in, Argmax am, double2* __restrict__ ws,
                                                       uint32_t* __restrict__ cnt) {
  Epi ep = ep_in;
  ep.mode = MODE;
  __shared__ double As[2][2][GBK][GBM + GPAD];
  __shared__ double Bs[2][2][GBK][GBN + GPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  // staging element tid + 256 i: A row (tid >> 4) + 16 i, k tid & 15 (16 lanes
  // read 256 contiguous bytes of a row); B row (tid >> 6) + 4 i, column
  // tid & 63 (a wave reads 1 KB of a row).  Measured on MI355X at the config-3
  // prefill shapes against 4 lanes per A row and 16 per B row, each lane 4
  // elements at a 64-byte stride: 48-50 -> 60 TFLOP/s.
  const int a_row = tid >> 4, a_k = tid & 15;
  const int b_k = tid >> 6, b_n = tid & 63;

  double2 ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + a_row + 16 * i, k = k0 + a_k;
      ra[i] = (m < M && k < kend) ? A[(long)m * lda + k] : make_double2(0.0, 0.0);
      const int kb = k0 + b_k + 4 * i, n = n0 + b_n;
      rb[i] = (kb < kend && n < N) ? Bm[(long)kb * ldb + n] : make_double2(0.0, 0.0);
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      As[st][0][a_k][a_row + 16 * i] = ra[i].x;
      As[st][1][a_k][a_row + 16 * i] = ra[i].y;
      Bs[st][0][b_k + 4 * i][b_n] = rb[i].x;
      Bs[st][1][b_k + 4 * i][b_n] = rb[i].y;
    }
  };

  v4d cr[2][2], ci[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) cr[i][j] = ci[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

  const int nk = kend > kbeg ? (kend - kbeg + GBK - 1) / GBK : 0;
  if (nk > 0) {
    gload(kbeg);
    sstore(0);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int st = it & 1;
    if (it + 1 < nk) gload(kbeg + (it + 1) * GBK);
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 4) {
      const int kr = kk + (lane >> 4);
      double ar[2], ai[2], br[2], bi[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ar[i] = As[st][0][kr][wm + 16 * i + (lane & 15)];
        ai[i] = As[st][1][kr][wm + 16 * i + (lane & 15)];
        br[i] = Bs[st][0][kr][wn + 16 * i + (lane & 15)];
        bi[i] = Bs[st][1][kr][wn + 16 * i + (lane & 15)];
      }
      // every tile's first two products before any tile's last two: an
      // accumulator's next MFMA comes 8 MFMAs after its previous one, not 2;
      // each accumulator still sums in the same order
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          cr[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[i], br[j], cr[i][j], 0, 0, 0);
          ci[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[i], bi[j], ci[i][j], 0, 0, 0);
        }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          cr[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(-ai[i], bi[j], cr[i][j], 0, 0, 0);
          ci[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ai[i], br[j], ci[i][j], 0, 0, 0);
        }
    }
    if (it + 1 < nk) sstore(st ^ 1);
    __syncthreads();
  }

  // Re values of the tile for the fused argmax, staged in the (now idle) As buffer
  double* stage = &As[0][0][0][0];  // [64][65]
  const bool argmax = am.part_v != nullptr;
  if (gridDim.z == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ml = wm + 16 * i + (lane >> 4) + 4 * r, nl = wn + 16 * j + (lane & 15);
          const int m = m0 + ml, n = n0 + nl;
          if (m < M && n < N) {
            const double re = apply_epi(ep, M, N, m, n, make_double2(cr[i][j][r], ci[i][j][r]));
            if (argmax) stage[ml * 65 + nl] = re;
          }
        }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + (lane >> 4) + 4 * r;
          const int n = n0 + wn + 16 * j + (lane & 15);
          if (m < M && n < N) st_dev(&ws[((long)blockIdx.z * M + m) * N + n], make_double2(cr[i][j][r], ci[i][j][r]));
        }
    if (!arrive_last(&cnt[blockIdx.y * gridDim.x + blockIdx.x], gridDim.z)) return;
    // thread t owns tile elements t + 256 i (row t/64 + 4i, column t%64); the
    // splits are summed in order, 16 independent loads in flight per split
    const int P = gridDim.z;
    const int nl = tid & 63, n = n0 + nl;
    double2 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = make_double2(0.0, 0.0);
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + (tid >> 6) + 4 * i;
        if (m < M && n < N) v[i] = cadd(v[i], ld_dev(&ws[((long)p * M + m) * N + n]));
      }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ml = (tid >> 6) + 4 * i, m = m0 + ml;
      if (m < M && n < N) {
        const double re = apply_epi(ep, M, N, m, n, v[i]);
        if (argmax) stage[ml * 65 + nl] = re;
      }
    }
  }
  if (!argmax) return;
  __syncthreads();
  // per-row (max, last index) over the tile's columns: wave w takes rows w, w+4, ...
  for (int ml = wave; ml < GBM; ml += 4) {
    const int m = m0 + ml, n = n0 + lane;
    if (m >= M) break;
    double bv = -INFINITY;
    int bi = -1;
    if (n < N) {
      const double v = stage[ml * 65 + lane];
      if (isnan(v)) atomicOr(am.err, (uint32_t)EB_ARGMAX_NAN);
      else bv = v, bi = n;
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
      am.part_v[(long)m * gridDim.x + blockIdx.x] = bv;
      am.part_i[(long)m * gridDim.x + blockIdx.x] = bi;
    }
  }
}

int launch_zgemm_mfma(hipStream_t st, dim3 grid, const double2* A, long lda, const double2* W, long ldw, int M, int N,
                      int K, int kchunk, const Epi& ep, const Argmax& am, double2* ws, uint32_t* cnt) {
  switch (ep.mode) {
    case EPI_STORE:
      MITOK_LAUNCH(k_zgemm_mfma<EPI_STORE>, grid, dim3(256), 0, st, A, lda, W, ldw, M, N, K, kchunk, ep, am, ws, cnt);
      return OK;
    case EPI_GELU:
      MITOK_LAUNCH(k_zgemm_mfma<EPI_GELU>, grid, dim3(256), 0, st, A, lda, W, ldw, M, N, K, kchunk, ep, am, ws, cnt);
      return OK;
    case EPI_RE:
      MITOK_LAUNCH(k_zgemm_mfma<EPI_RE>, grid, dim3(256), 0, st, A, lda, W, ldw, M, N, K, kchunk, ep, am, ws, cnt);
      return OK;
    case EPI_QKV:
      MITOK_LAUNCH(k_zgemm_mfma<EPI_QKV>, grid, dim3(256), 0, st, A, lda, W, ldw, M, N, K, kchunk, ep, am, ws, cnt);
      return OK;
    default:
      return ERR_ARG;  // split partials are for the skinny products
  }
}

}  // namespace mitok
