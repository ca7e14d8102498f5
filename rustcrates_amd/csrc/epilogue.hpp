// epilogue.hpp — what a product does with C[m][n] after the complex dot
// product (Epi in kernels.hpp): bias (utils/matrix.rs:615-625), GELU with pad
// rows zeroed (layer.rs:132-166, activation.rs:195-212,268-284), KV-cache
// append (masked_attention_head.rs:135-178) and Re-logits
// (data_converter.rs:244-256).  Shared by the product kernels and the
// resident decode loop (Acc: the access policy, common.hpp).
#pragma once

#include "rowops.hpp"

namespace mitok {

// ===========================================================================
// epilogue: returns Re of the stored value (used by the fused argmax)
// ===========================================================================
template <class Acc = AccPlain>
__device__ __forceinline__ double apply_epi(const Epi& ep, int M, int N, int m, int n, double2 v) {
  if (ep.bias) v = cadd(v, Acc::c(ep.bias + n));
  switch (ep.mode) {
    case EPI_STORE:
      if (ep.check_finite && !(isfinite(v.x) && isfinite(v.y))) atomicOr(ep.err, (uint32_t)EB_FFN_NONFINITE);
      Acc::st(ep.out + (long)m * ep.ldo + n, v);
      break;
    case EPI_GELU: {
      bool nan = false;
      if (ep.row_mask && Acc::c(ep.row_mask + m) == 0) v = make_double2(0.0, 0.0);  // activation.rs:268-284
      else v = gelu_nc(v, &nan);
      if (nan) atomicOr(ep.err, (uint32_t)EB_GELU_NAN);
      Acc::st(ep.out + (long)m * ep.ldo + n, v);
      break;
    }
    case EPI_RE:
      Acc::st(ep.out_re + (long)m * ep.ldo + n, v.x);
      if (ep.hist_re) Acc::st(ep.hist_re + ((long)Acc::cnt(ep.hist_cnt) * M + m) * N + n, v.x);
      break;
    case EPI_QKV: {
      if (n < ep.d) {
        Acc::st(ep.out + (long)m * ep.ldo + n, v);
        break;
      }
      const int part = n < 2 * ep.d ? 1 : 2;
      const int c = n - part * ep.d;
      const int h = c / ep.dh, e = c - h * ep.dh;
      const int b = m / ep.S, s = m - b * ep.S;
      if (ep.kv_row && Acc::kv(ep.kv_row, b) != s) break;  // cached branch: only the last token (masked_attention_head.rs:140-156)
      const int pos = (ep.kv_base ? Acc::kv(ep.kv_base, b) : 0) + (ep.kv_row ? 0 : s);
      if (pos >= ep.ctx) {
        atomicOr(ep.err, (uint32_t)EB_CTX_OVERFLOW);
        break;
      }
      double2* dst = part == 1 ? ep.kc : ep.vc;
      Acc::st(dst + (((long)b * ep.heads + h) * ep.ctx + pos) * ep.dh + e, v);
      break;
    }
  }
  return v.x;
}

}  // namespace mitok
