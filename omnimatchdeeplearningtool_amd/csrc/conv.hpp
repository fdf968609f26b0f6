// conv.hpp — host-side interface of the conv / BatchNorm path shared between
// the forward (conv.hip, eltwise.hip) and training (train.hip) entry points.
#pragma once

#include <hip/hip_runtime.h>

namespace omhip {

// Gather mode by kernel size: 0 = one 32-bit "tap outside the image" mask per
// pixel, 1 = a 64-bit mask, 2 = coordinate compares. Each mask mode keeps its
// top bit free (at most 31 / 63 taps): that bit is never an image tap, so it
// reads as "outside" for every pixel and serves as the code of rows past K.
__host__ __device__ constexpr int gatherMode(int taps) { return taps <= 31 ? 0 : (taps <= 63 ? 1 : 2); }

// out = act(BN(conv(x, w) + bias) + res) in one pass (bias, BN and res may be
// null); act 0 identity, 1 ReLU. `name` prefixes error messages. 0 or -1.
int conv2dFused(const char* name, const float* x, const float* w, const float* bias, const float* gamma,
                const float* beta, const float* mean, const float* var, float eps, const float* res, int act,
                float* out, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad);

// Stride-1 convolution onto an output grid: grid pixel (oh, ow), oh < Ho,
// ow < Wo, reads the window whose top-left tap is x[oh - padH][ow - padW]
// (negative pads start inside the image) and is written at
// (oh*oStride + oOffH, ow*oStride + oOffW) of an oH x oW output image; the
// output pixels off the grid are left untouched. No bias, BN or activation.
int conv2dToGrid(const char* name, const float* x, const float* w, float* out, int N, int Cin, int H, int W, int Cout,
                 int KH, int KW, int padH, int padW, int Ho, int Wo, int oH, int oW, int oStride, int oOffH,
                 int oOffW);

// The RGB stem geometry (3 input channels, 7x7, stride 2, pad 3, W a multiple
// of 4 up to 224) has a kernel of its own (conv_stem.hip); conv2dFused sends
// each batch chunk of that geometry there.
bool stemGeometry(int Cin, int W, int KH, int KW, int stride, int padH, int padW);

// out = act(BN(conv(x, w) + bias) + res) for the stem geometry, one chunk whose
// x, w and out views are at most 2^30 bytes. 0 or -1.
int convStem(const float* x, const float* w, const float* bias, const float* gamma, const float* beta,
             const float* mean, const float* var, float eps, const float* res, int act, float* out, int N, int H,
             int W, int Cout, int Ho, int Wo);

// gW[co][(ci*KH+kh)*KW+kw] = sum over images and output pixels of
// gradOutput[n][co][oh][ow] * x[n][ci][oh*stride-pad+kh][ow*stride-pad+kw]
// (overwrites gW). `name` prefixes error messages. 0 or -1.
int conv2dWeightGrad(const char* name, const float* x, const float* gO, float* gW, int N, int Cin, int H, int W,
                     int Cout, int KH, int KW, int stride, int pad);

// col[n][(c*KH+kh)*KW+kw][oh*Wo+ow] for every image of x (zero outside the image).
int im2colBatched(const float* x, float* col, int N, int Cin, int H, int W, int KH, int KW, int pad, int strd,
                  int Ho, int Wo);

// BatchNorm2d training forward (batch statistics, saved mean / inverse std,
// running averages, normalisation); saved pointers may be null.
int batchNorm2dTrain(const float* x, float* y, const float* gamma, const float* beta, float* runMean, float* runVar,
                     float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps, float momentum);

}  // namespace omhip
