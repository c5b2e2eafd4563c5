// Stock-op kernels of the full PP-DocLayoutV3 graph (net_ops.hip).
#pragma once

#include "ppdl_internal.h"

namespace ppdl {

// depthwise conv, w [C][K][K], out [C][OH][OW], + bias + act; x planes
// in_plane floats apart (>= IH*IW), out planes out_plane apart (>= OH*OW)
hipError_t dwconv(const float *x, const float *w, const float *b, float *out, int C, int IH, int IW, int K, int S,
                  int P, int act, int64_t in_plane, int64_t out_plane, hipStream_t s);
// 2x2 s1 max pool over x zero-padded at the right/bottom; out keeps [C][H][W]
hipError_t maxpool2_padend(const float *x, float *out, int C, int H, int W, hipStream_t s);
// out = interp(x) (+ add): nearest (bilinear = 0) or half-pixel bilinear
hipError_t interp(const float *x, const float *add, float *out, int C, int IH, int IW, int OH, int OW,
                  int bilinear, hipStream_t s);
// out = LN(a + b) over 256 features per token (b may be null); out_chw
// writes [256][T] instead of [T][256]
// slot = the device wall clock when the kernel runs (in-graph profiling)
hipError_t stamp(unsigned long long *slot, hipStream_t s);
// With row_mask set (no b), a row t with row_mask[t] == 0 is normalised as
// if it were row_fill ([256]).
hipError_t layernorm(const float *a, const float *b, const float *gamma, const float *beta, float *out, int T,
                     int out_chw, hipStream_t s, const float *row_mask = nullptr, const float *row_fill = nullptr);
// 8-head x 32 attention over token-major q/k/v (row strides in floats)
hipError_t attention(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv, float *out,
                     int ldo, int T, hipStream_t s);
hipError_t add(const float *a, const float *b, float *out, int64_t n, hipStream_t s);
hipError_t mul_rows(const float *x, const float *mask, float *out, int64_t T, int D, hipStream_t s);
// ref = sigmoid(delta + inv_sigmoid(ref)), or sigmoid(ref) when delta is null
hipError_t box_update(const float *delta, float *ref, int n, hipStream_t s);
hipError_t get_rows(const float *src, const int32_t *idx, float *out, int nrows, hipStream_t s);
hipError_t order_logits(const float *gp, float *out, int nq, int hd, float scale, hipStream_t s);
// in [rows][cols] -> out[c][r] with row stride ldo
hipError_t transpose(const float *in, float *out, int rows, int cols, int ldo, hipStream_t s);

}  // namespace ppdl
