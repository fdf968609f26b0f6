// ref_bind.cpp — C entry points over the reference's own CPUBackend module
// (src/hal/om.hal.cpu_backend.ixx, which imports src/hal/om.hal.simd.ixx),
// compiled from the reference sources in place by oracle/Makefile into
// oracle/_ref/libomref_reference.so. Used only to check the oracle restatement
// (omref.cpp) and as the timed CPU baseline; nothing in libomhip touches it.
#include <cstddef>
#include <cstdint>
import om.hal.cpu_backend;

extern "C" {
void refMatmul(const float* a, const float* b, float* c, int m, int k, int n) { om::CPUBackend::matmul(a, b, c, m, k, n); }
void refBatchedMatmul(const float* a, const float* b, float* c, int batch, int m, int k, int n) {
    om::CPUBackend::batchedMatmul(a, b, c, batch, m, k, n);
}
void refTranspose2d(const float* a, float* b, int rows, int cols) { om::CPUBackend::transpose2d(a, b, rows, cols); }
void refIm2col(const float* x, int cin, int h, int w, int kh, int kw, int ph, int pw, int sh, int sw, float* col) {
    om::CPUBackend::im2col(x, cin, h, w, kh, kw, ph, pw, sh, sw, col);
}
void refConv2d(const float* x, const float* w, const float* bias, float* out, int n, int cin, int h, int wd, int cout,
               int kh, int kw, int stride, int pad) {
    om::CPUBackend::conv2d(x, w, bias, out, n, cin, h, wd, cout, kh, kw, stride, pad);
}
void refBatchNorm2d(const float* x, float* y, const float* g, const float* b, float* rm, float* rv, float* sm,
                    float* si, int n, int c, int h, int w, float eps, float mom, int training) {
    om::CPUBackend::batchNorm2d(x, y, g, b, rm, rv, sm, si, n, c, h, w, eps, mom, training != 0);
}
void refRelu(const float* x, float* y, size_t n) { om::CPUBackend::relu(x, y, n); }
void refReluBackward(const float* x, const float* g, float* gi, size_t n) { om::CPUBackend::reluBackward(x, g, gi, n); }
void refAddBias(const float* a, const float* bias, float* out, int batch, int cols) {
    om::CPUBackend::addBias(a, bias, out, batch, cols);
}
void refConv2dBackwardInput(const float* gO, const float* w, float* gI, int n, int cin, int h, int wd, int cout, int kh,
                            int kw, int stride, int pad) {
    om::CPUBackend::conv2dBackwardInput(gO, w, gI, n, cin, h, wd, cout, kh, kw, stride, pad);
}
void refConv2dBackwardWeight(const float* x, const float* gO, float* gW, float* gB, int n, int cin, int h, int wd,
                             int cout, int kh, int kw, int stride, int pad) {
    om::CPUBackend::conv2dBackwardWeight(x, gO, gW, gB, n, cin, h, wd, cout, kh, kw, stride, pad);
}
void refBatchNorm2dBackward(const float* gO, const float* x, const float* mean, const float* invStd, const float* g,
                            float* gI, float* gG, float* gB, int n, int c, int h, int w) {
    om::CPUBackend::batchNorm2dBackward(gO, x, mean, invStd, g, gI, gG, gB, n, c, h, w);
}
void refMaxPool2d(const float* x, float* y, int* idx, int n, int c, int h, int w, int kh, int kw, int stride, int pad) {
    om::CPUBackend::maxPool2d(x, y, idx, n, c, h, w, kh, kw, stride, pad);
}
void refMaxPool2dBackward(const float* gO, const int* idx, float* gI, int n, int c, int ho, int wo, int h, int w) {
    om::CPUBackend::maxPool2dBackward(gO, idx, gI, n, c, ho, wo, h, w);
}
void refAvgPool2d(const float* x, float* y, int n, int c, int h, int w, int kh, int kw, int stride, int pad) {
    om::CPUBackend::avgPool2d(x, y, n, c, h, w, kh, kw, stride, pad);
}
void refAvgPool2dBackward(const float* gO, float* gI, int n, int c, int h, int w, int ho, int wo, int kh, int kw,
                          int stride, int pad) {
    om::CPUBackend::avgPool2dBackward(gO, gI, n, c, h, w, ho, wo, kh, kw, stride, pad);
}
void refAdaptiveAvgPool2d(const float* x, float* y, int n, int c, int h, int w, int oh, int ow) {
    om::CPUBackend::adaptiveAvgPool2d(x, y, n, c, h, w, oh, ow);
}
void refAdaptiveAvgPool2dBackward(const float* gO, float* gI, int n, int c, int h, int w, int oh, int ow) {
    om::CPUBackend::adaptiveAvgPool2dBackward(gO, gI, n, c, h, w, oh, ow);
}
void refAdd(const float* a, const float* b, float* out, size_t n) { om::CPUBackend::add(a, b, out, n); }
float refSum(const float* x, size_t n) { return om::CPUBackend::sum(x, n); }
void refSoftmax(const float* in, float* out, int rows, int cols) { om::CPUBackend::softmax(in, out, rows, cols); }
float refCrossEntropy(const float* p, const float* t, int rows, int cols) {
    return om::CPUBackend::crossEntropy(p, t, rows, cols);
}
void refCrossEntropySoftmaxBackward(const float* s, const float* t, float* g, int rows, int cols) {
    om::CPUBackend::crossEntropySoftmaxBackward(s, t, g, rows, cols);
}
}
