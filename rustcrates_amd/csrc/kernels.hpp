// kernels.hpp — launch wrappers of the gfx950 kernels (kernels.hip).
//
// Every wrapper enqueues on `st` and never synchronises or allocates, so the
// decode step built from them can be captured into a HIP graph.
#pragma once

#include "common.hpp"

namespace mitok {

// ---- GEMM epilogue: what happens to C[m][n] after the complex dot product ----
enum EpiMode : int {
  EPI_STORE = 0,  // out[m][n] = v (+bias); optional non-finite check (FFN output)
  EPI_GELU = 1,   // out[m][n] = mask[m] ? gelu(v + bias) : 0 (layer.rs:132-166)
  EPI_RE = 2,     // out_re[m][n] = Re(v + bias) (logits, data_converter.rs:244-256)
  EPI_QKV = 3,    // columns [q | k | v] of all heads: q -> out, k/v -> KV cache
};

struct Epi {
  int mode = EPI_STORE;
  const double2* bias = nullptr;  // [N]
  double2* out = nullptr;         // STORE / GELU / QKV(q part)
  double* out_re = nullptr;       // RE
  long ldo = 0;
  const uint32_t* row_mask = nullptr;  // GELU: rows with mask 0 become 0
  int check_finite = 0;
  uint32_t* err = nullptr;
  // EPI_QKV: row m = b * S + s
  int d = 0, dh = 0, heads = 0, S = 1;
  double2* kc = nullptr;  // [B][heads][ctx][dh]
  double2* vc = nullptr;
  int ctx = 0;
  const int* kv_base = nullptr;  // [B] cache position of row s = 0 (null: 0)
  const int* kv_row = nullptr;   // [B] only this row is appended (null: every row)
};

// GEMM C[M][N] = A[M][K] * B[K][N] (complex, row-major), then the epilogue.
// Small M uses a bandwidth GEMV, larger M the MFMA-tiled kernel; split-K
// partial sums go to `ws`.  gemm_ws_bytes() is the workspace it needs.
size_t gemm_ws_bytes(int M, int N, int K, int mode);
void gemm(hipStream_t st, int M, int N, int K, const double2* A, long lda, const double2* B, long ldb, const Epi& ep,
          void* ws);

// ---- attention ----
struct Attn {
  const double2* q = nullptr;  // [B*S][ldq]; head h at column h*dh
  long ldq = 0;
  const double2* kc = nullptr;  // [B][H][ctx][dh]
  const double2* vc = nullptr;
  int ctx = 0;
  const int* kv_len = nullptr;  // [B]: keys = kv_len[b] + T_add (null: T_const)
  int T_add = 0, T_const = 0;
  int T_max = 0;                // upper bound on keys (sizing)
  const double* bias_re = nullptr;  // [H][mc][mc] Re(bias_pos)
  int mc = 0;
  const uint32_t* row_mask = nullptr;  // [B*S]
  double2* out = nullptr;              // [B*S][ldo], head h at column h*dh
  long ldo = 0;
  int B = 0, S = 0, H = 0, dh = 0;
  double scale = 1.0;
};
// One query row per block (prefill and the general reference case).
void attention_rows(hipStream_t st, const Attn& a);
// Split-key decode (S == 1): partial softmax per key chunk, then a combine.
size_t attention_decode_ws_bytes(int B, int H, int dh, int T_max);
void attention_decode(hipStream_t st, const Attn& a, void* ws);

// ---- row kernels ----
void embed(hipStream_t st, const double2* table, int V, int d, const uint32_t* ids, int rows, double2* out,
           uint32_t* err);
// positions per row (pos != null) or per sequence from kv_len (S == 1 decode)
void rope(hipStream_t st, double2* x, int rows, int d, const double2* cs_table, int max_pos, const int* pos,
          const int* kv_len, uint32_t* err);
void layernorm(hipStream_t st, const double2* x, const double2* before, double2* out, int rows, int d, double eps,
               const double2* gamma, const double2* beta);
void gather_rows(hipStream_t st, const double2* src, int S, int d, const uint32_t* lens, int B, double2* dst);
// argmax per row with last-index ties; ids[b]; optional history append and kv advance
void argmax_rows(hipStream_t st, const double* logits, int rows, int V, uint32_t* ids, uint32_t* hist, int hist_stride,
                 int* hist_cnt, int* kv_len, int advance_kv, uint32_t* err);
void softmax_rows(hipStream_t st, const double2* logits, int rows, int S, int V, const uint32_t* row_mask, int mode,
                  double* out);
void store_logits(hipStream_t st, const double* logits, int rows, int V, double* hist, const int* hist_cnt);

// ---- initialisation ----
void fill_seeded(hipStream_t st, double2* dst, int rows, int cols, long ld, uint64_t key, double lim);
void fill_seeded_re(hipStream_t st, double* dst, int rows, int cols, long ld, uint64_t key, double lim);
void fill_const(hipStream_t st, double2* dst, size_t n, double2 v);
void fill_int(hipStream_t st, int* dst, size_t n, int v);
void fill_u32(hipStream_t st, uint32_t* dst, size_t n, uint32_t v);
void copy_re(hipStream_t st, const double2* src, double* dst, size_t n);

}  // namespace mitok
