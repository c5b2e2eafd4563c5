// Bandwidth kernels: op 5 bias+act and the F32 im2col in ggml's layout.
#include <algorithm>

#include "device_math.h"

namespace ppdl {
namespace {

// out[i] = act(in[i] + bias[i / plane])   (patches/ggml-ppdl.patch:417-432)
// Vector path: 4 consecutive elements share one bias when plane % 4 == 0.
__global__ __launch_bounds__(256) void k_bias_act4(const float4 *__restrict__ in,
                                                   const float *__restrict__ bias,
                                                   float4 *__restrict__ out, int64_t n4,
                                                   int64_t plane4, int act) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float b = bias[i / plane4];
        float4 v = in[i];
        v.x = act_f(v.x + b, act);
        v.y = act_f(v.y + b, act);
        v.z = act_f(v.z + b, act);
        v.w = act_f(v.w + b, act);
        out[i] = v;
    }
}

__global__ __launch_bounds__(256) void k_bias_act1(const float *__restrict__ in,
                                                   const float *__restrict__ bias,
                                                   float *__restrict__ out, int64_t n,
                                                   int64_t plane, int act) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = act_f(in[i] + bias[i / plane], act);
}

// im2col through an LDS tile of 64 pixels x 64 k: the gather phase walks
// pixels fastest (consecutive output columns read consecutive input columns
// for stride 1), the store phase walks k fastest (dst rows are k-contiguous).
constexpr int kIT = 64;

__global__ __launch_bounds__(256) void k_im2col(const float *__restrict__ x, float *__restrict__ dst,
                                                int64_t IW, int64_t IH, int64_t OW, int64_t OH,
                                                int64_t KW, int64_t KH, int64_t IC, int64_t npix,
                                                int64_t ch_stride, int64_t img_stride, int s0,
                                                int s1, int p0, int p1, int d0, int d1) {
    __shared__ float tile[kIT][kIT + 1];
    const int64_t KK = KH * KW, KT = IC * KK;
    const int64_t pix0 = (int64_t)blockIdx.x * kIT;
    const int64_t k0 = (int64_t)blockIdx.y * kIT;
    const int tid = threadIdx.x;

    // gather: thread -> (k row = tid/64 + 4e, pixel = tid%64)
    {
        const int lp = tid & 63;
        const int64_t pix = pix0 + lp;
        int64_t ow = 0, oh = 0, img = 0;
        if (pix < npix) {
            ow = pix % OW;
            const int64_t z = pix / OW;
            oh = z % OH;
            img = z / OH;
        }
        for (int r = tid >> 6; r < kIT; r += 4) {
            const int64_t k = k0 + r;
            float v = 0.0f;
            if (pix < npix && k < KT) {
                const int64_t ic = k / KK, rem = k - ic * KK;
                const int64_t kh = rem / KW, kw = rem - kh * KW;
                const int64_t iy = oh * s1 + kh * d1 - p1;
                const int64_t ix = ow * s0 + kw * d0 - p0;
                if (iy >= 0 && iy < IH && ix >= 0 && ix < IW)
                    v = x[ic * ch_stride + img * img_stride + iy * IW + ix];
            }
            tile[r][lp] = v;
        }
    }
    __syncthreads();
    // store: thread -> (pixel = tid/64 + 4e, k = tid%64)
    {
        const int lk = tid & 63;
        const int64_t k = k0 + lk;
        if (k < KT) {
            for (int r = tid >> 6; r < kIT; r += 4) {
                const int64_t pix = pix0 + r;
                if (pix < npix) dst[pix * KT + k] = tile[lk][r];
            }
        }
    }
}

}  // namespace

hipError_t bias_act(const float *in, const float *bias, float *out, int64_t n, int64_t plane,
                    int act, hipStream_t s) {
    const bool vec = (n % 4 == 0) && (plane % 4 == 0) && ((((uintptr_t)in) & 15) == 0) &&
                     ((((uintptr_t)out) & 15) == 0);
    if (vec) {
        const int64_t n4 = n / 4;
        const unsigned blocks = (unsigned)std::min<int64_t>((n4 + 255) / 256, 1 << 16);
        hipLaunchKernelGGL(k_bias_act4, dim3(blocks), dim3(256), 0, s, (const float4 *)in, bias,
                           (float4 *)out, n4, plane / 4, act);
    } else {
        const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 1 << 16);
        hipLaunchKernelGGL(k_bias_act1, dim3(blocks), dim3(256), 0, s, in, bias, out, n, plane, act);
    }
    return hipGetLastError();
}

hipError_t im2col_ggml(const float *x, float *dst, int64_t IW, int64_t IH, int64_t OW, int64_t OH,
                       int64_t KW, int64_t KH, int64_t IC, int64_t N, int64_t ch_stride,
                       int64_t img_stride, int s0, int s1, int p0, int p1, int d0, int d1,
                       hipStream_t s) {
    const int64_t npix = N * OH * OW;
    const int64_t KT = IC * KH * KW;
    const dim3 grid((unsigned)((npix + kIT - 1) / kIT), (unsigned)((KT + kIT - 1) / kIT));
    hipLaunchKernelGGL(k_im2col, grid, dim3(256), 0, s, x, dst, IW, IH, OW, OH, KW, KH, IC, npix,
                       ch_stride, img_stride, s0, s1, p0, p1, d0, d1);
    return hipGetLastError();
}

}  // namespace ppdl
