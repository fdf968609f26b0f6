// conv.hpp — host-side interface of the conv / BatchNorm path shared between
// the forward (conv.hip, eltwise.hip) and training (train.hip) entry points.
#pragma once

namespace omhip {

// out = act(BN(conv(x, w) + bias) + res) in one pass (bias, BN and res may be
// null); act 0 identity, 1 ReLU. `name` prefixes error messages. 0 or -1.
int conv2dFused(const char* name, const float* x, const float* w, const float* bias, const float* gamma,
                const float* beta, const float* mean, const float* var, float eps, const float* res, int act,
                float* out, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad);

// col[n][(c*KH+kh)*KW+kw][oh*Wo+ow] for every image of x (zero outside the image).
int im2colBatched(const float* x, float* col, int N, int Cin, int H, int W, int KH, int KW, int pad, int strd,
                  int Ho, int Wo);

// BatchNorm2d training forward (batch statistics, saved mean / inverse std,
// running averages, normalisation); saved pointers may be null.
int batchNorm2dTrain(const float* x, float* y, const float* gamma, const float* beta, float* runMean, float* runVar,
                     float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps, float momentum);

}  // namespace omhip
