// omref.cpp — the ORACLE: a CPU restatement of the reference CPUBackend hot
// path (rhine311014/OmniMatchDeeplearningTool, src/hal/om.hal.cpu_backend.ixx
// and src/hal/om.hal.simd.ixx). Test infrastructure only: the parity tests,
// the smoke check and the bench's CPU baseline leg load it as the checker;
// libomhip never links or calls it.
//
// Every function follows the cited reference lines, including evaluation
// order, so its results are bit-identical to the reference CPUBackend built
// with clang (-O3 -mavx2 -mfma, which contracts a*b+c into one fma):
//   - matmul: each C[i][j] is the fma chain acc = fma(A[i][k], B[k][j], acc)
//     over k = 0..K-1 from acc = 0 — the 4x8 AVX2 tile (simd.ixx:102-124), the
//     1x8 row remainder (:135-144) and the contracted scalar column remainder
//     (:149-157) all evaluate that chain; the AVX2 restatement below keeps the
//     4x8 register tile and the OpenMP 4-row blocking (cpu_backend.ixx:256-265)
//     so it is also a fair timing of the reference path;
//   - conv2d: per image im2col -> matmul -> separate bias add (:619-658);
//   - batchNorm2d: invStd = 1/sqrt(var+eps) in fp32, y = fma(gamma, (x-mean)*invStd, beta)
//     (:781-842);
//   - relu: x > 0 ? x : 0 (:317-332, simd.ixx:248-274).
// Each extern "C" entry below names its reference lines.
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>
#include <algorithm>
#include <omp.h>
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define OMREF_AVX2 1
#endif

namespace {

// simd.ixx:72-170 — C[M,N] = A[M,K] B[K,N]; C zeroed first (simd.ixx:81).
void matmulTile(const float* A, const float* B, float* C, int M, int K, int N) {
    std::memset(C, 0, sizeof(float) * (size_t)M * N);
#ifdef OMREF_AVX2
    const int N8 = N & ~7, M4 = M & ~3;
    for (int j = 0; j < N8; j += 8) {
        for (int i = 0; i < M4; i += 4) {
            __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
            __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
            for (int k = 0; k < K; ++k) {
                const __m256 b = _mm256_loadu_ps(B + (size_t)k * N + j);
                s0 = _mm256_fmadd_ps(_mm256_set1_ps(A[(size_t)(i + 0) * K + k]), b, s0);
                s1 = _mm256_fmadd_ps(_mm256_set1_ps(A[(size_t)(i + 1) * K + k]), b, s1);
                s2 = _mm256_fmadd_ps(_mm256_set1_ps(A[(size_t)(i + 2) * K + k]), b, s2);
                s3 = _mm256_fmadd_ps(_mm256_set1_ps(A[(size_t)(i + 3) * K + k]), b, s3);
            }
            _mm256_storeu_ps(C + (size_t)(i + 0) * N + j, s0);
            _mm256_storeu_ps(C + (size_t)(i + 1) * N + j, s1);
            _mm256_storeu_ps(C + (size_t)(i + 2) * N + j, s2);
            _mm256_storeu_ps(C + (size_t)(i + 3) * N + j, s3);
        }
        for (int i = M4; i < M; ++i) {
            __m256 s = _mm256_setzero_ps();
            for (int k = 0; k < K; ++k)
                s = _mm256_fmadd_ps(_mm256_set1_ps(A[(size_t)i * K + k]), _mm256_loadu_ps(B + (size_t)k * N + j), s);
            _mm256_storeu_ps(C + (size_t)i * N + j, s);
        }
    }
    for (int i = 0; i < M; ++i)
        for (int j = N8; j < N; ++j) {
            float v = 0.f;
            for (int k = 0; k < K; ++k) v = std::fma(A[(size_t)i * K + k], B[(size_t)k * N + j], v);
            C[(size_t)i * N + j] = v;
        }
#else
    // Same per-element fma chain without vector registers.
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float v = 0.f;
            for (int k = 0; k < K; ++k) v = std::fma(A[(size_t)i * K + k], B[(size_t)k * N + j], v);
            C[(size_t)i * N + j] = v;
        }
#endif
}

}  // namespace

extern "C" {

// cpu_backend.ixx:65-77
void omrefFillValue(float* p, size_t n, float v) { for (size_t i = 0; i < n; ++i) p[i] = v; }

// cpu_backend.ixx:239-286: null pointers or non-positive dims zero C (246-251);
// M >= 4 -> OpenMP over 4-row blocks, each a 4-row matmulAVX2 (256-265); M < 4 -> one call (269).
void omrefMatmul(const float* A, const float* B, float* C, int M, int K, int N) {
    if (!A || !B || !C || M <= 0 || K <= 0 || N <= 0) {
        if (C && M > 0 && N > 0) std::memset(C, 0, sizeof(float) * (size_t)M * N);
        return;
    }
    if (M >= 4) {
#pragma omp parallel for schedule(dynamic, 1)
        for (int b = 0; b < M; b += 4) {
            const int rows = std::min(4, M - b);
            matmulTile(A + (size_t)b * K, B, C + (size_t)b * N, rows, K, N);
        }
        return;
    }
    matmulTile(A, B, C, M, K, N);
}

// cpu_backend.ixx:1535-1539
void omrefTranspose2d(const float* A, float* B, int rows, int cols) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) B[(size_t)c * rows + r] = A[(size_t)r * cols + c];
}

// cpu_backend.ixx:1520-1532 (the batch loop; the per-batch results do not
// depend on the OpenMP clause, which only changes which thread runs a batch)
void omrefBatchedMatmul(const float* A, const float* B, float* C, int batch, int M, int K, int N) {
    for (int b = 0; b < batch; ++b)
        omrefMatmul(A + (size_t)b * M * K, B + (size_t)b * K * N, C + (size_t)b * M * N, M, K, N);
}

// transpose2d + matmul: the composition the reference uses for A x B^T
// (autograd.ixx:261-273; vit.ixx:175-176 via tensorTranspose2dBatched).
void omrefMatmulTransB(const float* A, const float* Bnk, float* C, int M, int K, int N) {
    std::vector<float> bt((size_t)K * N);
    omrefTranspose2d(Bnk, bt.data(), N, K);
    omrefMatmul(A, bt.data(), C, M, K, N);
}

// transpose2d + matmul for A^T x B (autograd.ixx:276-286).
void omrefMatmulTransA(const float* Akm, const float* B, float* C, int M, int K, int N) {
    std::vector<float> at((size_t)M * K);
    omrefTranspose2d(Akm, at.data(), K, M);
    omrefMatmul(at.data(), B, C, M, K, N);
}

void omrefBatchedMatmulTransB(const float* A, const float* B, float* C, int batch, int M, int K, int N) {
    for (int b = 0; b < batch; ++b)
        omrefMatmulTransB(A + (size_t)b * M * K, B + (size_t)b * N * K, C + (size_t)b * M * N, M, K, N);
}

// MatMulBackward::backward (autograd.ixx:226-290): dA = G[M,N] x B^T, dB = A^T x G,
// each an explicit transpose followed by matmul (both always computed).
void omrefMatmulBackward(const float* G, const float* A, const float* B, float* dA, float* dB, int M, int K, int N) {
    std::vector<float> bt((size_t)N * K), at((size_t)K * M);
    for (int i = 0; i < K; ++i)
        for (int j = 0; j < N; ++j) bt[(size_t)j * K + i] = B[(size_t)i * N + j];
    omrefMatmul(G, bt.data(), dA, M, N, K);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < K; ++j) at[(size_t)j * M + i] = A[(size_t)i * K + j];
    omrefMatmul(at.data(), G, dB, K, M, N);
}

// cpu_backend.ixx:544-575
void omrefIm2col(const float* x, int Cin, int H, int W, int KH, int KW, int ph, int pw, int sh, int sw, float* col) {
    const int Ho = (H + 2 * ph - KH) / sh + 1, Wo = (W + 2 * pw - KW) / sw + 1;
    const int cols = Ho * Wo;
    for (int c = 0; c < Cin; ++c)
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw) {
                const int row = (c * KH + kh) * KW + kw;
                for (int oh = 0; oh < Ho; ++oh)
                    for (int ow = 0; ow < Wo; ++ow) {
                        const int ih = oh * sh - ph + kh, iw = ow * sw - pw + kw;
                        col[(size_t)row * cols + oh * Wo + ow] =
                            (ih >= 0 && ih < H && iw >= 0 && iw < W) ? x[((size_t)c * H + ih) * W + iw] : 0.f;
                    }
            }
}

// cpu_backend.ixx:619-658: per image im2col -> matmul(W[Cout,K], col) -> bias add.
void omrefConv2d(const float* x, const float* w, const float* bias, float* out, int N, int Cin, int H, int W,
                 int Cout, int KH, int KW, int stride, int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    const int rows = Cin * KH * KW, cols = Ho * Wo;
    std::vector<float> col((size_t)rows * cols);
    for (int n = 0; n < N; ++n) {
        omrefIm2col(x + (size_t)n * Cin * H * W, Cin, H, W, KH, KW, pad, pad, stride, stride, col.data());
        float* o = out + (size_t)n * Cout * cols;
        omrefMatmul(w, col.data(), o, Cout, rows, cols);
        if (bias)
            for (int c = 0; c < Cout; ++c)
                for (int i = 0; i < cols; ++i) o[(size_t)c * cols + i] += bias[c];
    }
}

// cpu_backend.ixx:781-842 (training 796-822, eval 823-830, normalize 832-840).
void omrefBatchNorm2d(const float* x, float* y, const float* gamma, const float* beta, float* runMean, float* runVar,
                      float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps, float momentum,
                      int training) {
    const int S = H * W;
    const int cnt = N * S;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < C; ++c) {
        float mean = 0.f, var = 0.f;
        if (training) {
            for (int n = 0; n < N; ++n)
                for (int s = 0; s < S; ++s) mean += x[((size_t)n * C + c) * S + s];
            mean /= (float)cnt;
            for (int n = 0; n < N; ++n)
                for (int s = 0; s < S; ++s) {
                    const float d = x[((size_t)n * C + c) * S + s] - mean;
                    var = std::fma(d, d, var);
                }
            var /= (float)cnt;
            if (savedMean) savedMean[c] = mean;
            if (savedInvStd) savedInvStd[c] = 1.0f / std::sqrt(var + eps);
            runMean[c] = std::fma(1.0f - momentum, runMean[c], momentum * mean);
            runVar[c] = std::fma(1.0f - momentum, runVar[c], momentum * var);
        } else {
            mean = runMean[c];
            var = runVar[c];
            if (savedMean) savedMean[c] = mean;
            if (savedInvStd) savedInvStd[c] = 1.0f / std::sqrt(var + eps);
        }
        const float inv = 1.0f / std::sqrt(var + eps);
        for (int n = 0; n < N; ++n)
            for (int s = 0; s < S; ++s) {
                const size_t i = ((size_t)n * C + c) * S + s;
                y[i] = std::fma(gamma[c], (x[i] - mean) * inv, beta[c]);
            }
    }
}

// cpu_backend.ixx:317-332 / simd.ixx:248-274
void omrefRelu(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = x[i] > 0.f ? x[i] : 0.f;
}

// cpu_backend.ixx:337-346
void omrefReluBackward(const float* x, const float* g, float* gi, size_t n) {
    for (size_t i = 0; i < n; ++i) gi[i] = x[i] > 0.f ? g[i] : 0.f;
}

// cpu_backend.ixx:433-440 (row broadcast)
void omrefAddBias(const float* A, const float* bias, float* out, int batch, int cols) {
    for (int b = 0; b < batch; ++b)
        for (int j = 0; j < cols; ++j) out[(size_t)b * cols + j] = A[(size_t)b * cols + j] + bias[j];
}

// conv2d -> batchNorm2d(eval) -> relu: the reference 3-call chain that the
// fused entry replaces (tensor_ops.ixx:672-833, :511-536).
void omrefConvBnRelu(const float* x, const float* w, const float* bias, const float* gamma, const float* beta,
                     const float* mean, const float* var, float eps, int act, float* out, int N, int Cin, int H,
                     int W, int Cout, int KH, int KW, int stride, int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    const size_t n = (size_t)N * Cout * Ho * Wo;
    std::vector<float> t(n);
    omrefConv2d(x, w, bias, t.data(), N, Cin, H, W, Cout, KH, KW, stride, pad);
    if (gamma) {
        std::vector<float> m(mean, mean + Cout), v(var, var + Cout);
        omrefBatchNorm2d(t.data(), t.data(), gamma, beta, m.data(), v.data(), nullptr, nullptr, N, Cout, Ho, Wo, eps,
                         0.1f, 0);
    }
    if (act == 1) omrefRelu(t.data(), out, n);
    else std::memcpy(out, t.data(), n * sizeof(float));
}

// FP16Converter::floatToHalf (src/engine/om.engine.fp16.ixx:36-100): the
// reference's software converter TRUNCATES the mantissa (>>13) and flushes
// fp32 subnormals to signed zero. Restated for documentation of the rounding
// ---- training path and pooling -------------------------------------------------

// cpu_backend.ixx:581-607 — scatter-add of a column matrix back onto one image.
void omrefCol2im(const float* col, int Cin, int H, int W, int KH, int KW, int ph, int pw, int sh, int sw, float* x) {
    const int Ho = (H + 2 * ph - KH) / sh + 1, Wo = (W + 2 * pw - KW) / sw + 1;
    const int cols = Ho * Wo;
    for (int c = 0; c < Cin; ++c)
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw) {
                const int row = (c * KH + kh) * KW + kw;
                for (int oh = 0; oh < Ho; ++oh)
                    for (int ow = 0; ow < Wo; ++ow) {
                        const int ih = oh * sh - ph + kh, iw = ow * sw - pw + kw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W)
                            x[((size_t)c * H + ih) * W + iw] += col[(size_t)row * cols + oh * Wo + ow];
                    }
            }
}

// cpu_backend.ixx:666-705 — gradInput = col2im(W^T x gradOutput), per image.
void omrefConv2dBackwardInput(const float* gO, const float* w, float* gI, int N, int Cin, int H, int W, int Cout,
                              int KH, int KW, int stride, int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    const int rows = Cin * KH * KW, cols = Ho * Wo;
    std::memset(gI, 0, (size_t)N * Cin * H * W * sizeof(float));
    std::vector<float> wt((size_t)rows * Cout), col((size_t)rows * cols);
    omrefTranspose2d(w, wt.data(), Cout, rows);
    for (int n = 0; n < N; ++n) {
        omrefMatmul(wt.data(), gO + (size_t)n * Cout * cols, col.data(), rows, Cout, cols);
        omrefCol2im(col.data(), Cin, H, W, KH, KW, pad, pad, stride, stride, gI + (size_t)n * Cin * H * W);
    }
}

// cpu_backend.ixx:710-772 — gradWeight = sum_n gradOutput[n] x im2col(x[n])^T,
// gradBias[co] = sum_n (sum_hw gradOutput[n][co][hw]).
void omrefConv2dBackwardWeight(const float* x, const float* gO, float* gW, float* gB, int N, int Cin, int H, int W,
                               int Cout, int KH, int KW, int stride, int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    const int rows = Cin * KH * KW, cols = Ho * Wo;
    const size_t wsz = (size_t)Cout * rows;
    std::memset(gW, 0, wsz * sizeof(float));
    if (gB) std::memset(gB, 0, (size_t)Cout * sizeof(float));
    std::vector<float> col((size_t)rows * cols), colT((size_t)rows * cols), tmp(wsz);
    for (int n = 0; n < N; ++n) {
        omrefIm2col(x + (size_t)n * Cin * H * W, Cin, H, W, KH, KW, pad, pad, stride, stride, col.data());
        omrefTranspose2d(col.data(), colT.data(), rows, cols);
        omrefMatmul(gO + (size_t)n * Cout * cols, colT.data(), tmp.data(), Cout, cols, rows);
        for (size_t i = 0; i < wsz; ++i) gW[i] += tmp[i];
        if (gB) {
            const float* g = gO + (size_t)n * Cout * cols;
            for (int co = 0; co < Cout; ++co) {
                float b = 0.f;
                for (int hw = 0; hw < cols; ++hw) b += g[(size_t)co * cols + hw];
                gB[co] += b;
            }
        }
    }
}

// cpu_backend.ixx:847-890 — per channel: gradGamma = sum(dy * xhat), gradBeta = sum(dy),
// dx = gamma*invStd/cnt * (cnt*dy - gradBeta - xhat*gradGamma) (clang contracts the
// sums and the bracket into fmas).
void omrefBatchNorm2dBackward(const float* gO, const float* x, const float* mean, const float* invStd,
                              const float* gamma, float* gI, float* gG, float* gBeta, int N, int C, int H, int W) {
    const int S = H * W;
    const int cnt = N * S;
    const float invCnt = 1.0f / (float)cnt;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < C; ++c) {
        const float m = mean[c], is = invStd[c], g = gamma[c];
        float sg = 0.f, sb = 0.f;
        for (int n = 0; n < N; ++n)
            for (int s = 0; s < S; ++s) {
                const size_t i = ((size_t)n * C + c) * S + s;
                const float xh = (x[i] - m) * is;
                sg = std::fma(gO[i], xh, sg);
                sb += gO[i];
            }
        gG[c] = sg;
        gBeta[c] = sb;
        for (int n = 0; n < N; ++n)
            for (int s = 0; s < S; ++s) {
                const size_t i = ((size_t)n * C + c) * S + s;
                const float xh = (x[i] - m) * is;
                gI[i] = g * is * invCnt * std::fma(-xh, sg, std::fma((float)cnt, gO[i], -sb));
            }
    }
}

// cpu_backend.ixx:897-934 — max over the window (strictly greater wins, so the
// first maximum in kh, kw order is kept); the index is the flat input index, -1
// for a window entirely in the padding (output -1e30).
void omrefMaxPool2d(const float* x, float* y, int* idx, int N, int C, int H, int W, int KH, int KW, int stride,
                    int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    for (int nc = 0; nc < N * C; ++nc)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow) {
                float best = -1e30f;
                int bi = -1;
                for (int kh = 0; kh < KH; ++kh)
                    for (int kw = 0; kw < KW; ++kw) {
                        const int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                            const int ii = (nc * H + ih) * W + iw;
                            if (x[ii] > best) {
                                best = x[ii];
                                bi = ii;
                            }
                        }
                    }
                const size_t o = ((size_t)nc * Ho + oh) * Wo + ow;
                y[o] = best;
                idx[o] = bi;
            }
}

// cpu_backend.ixx:937-955 — scatter-add through the saved indices in output order.
void omrefMaxPool2dBackward(const float* gO, const int* idx, float* gI, int N, int C, int Ho, int Wo, int H, int W) {
    const size_t nin = (size_t)N * C * H * W, nout = (size_t)N * C * Ho * Wo;
    for (size_t i = 0; i < nin; ++i) gI[i] = 0.f;
    for (size_t i = 0; i < nout; ++i)
        if (idx[i] >= 0) gI[idx[i]] += gO[i];
}

// cpu_backend.ixx:958-990 — window sum over the valid taps divided by KH*KW
// (padding counts in the divisor).
void omrefAvgPool2d(const float* x, float* y, int N, int C, int H, int W, int KH, int KW, int stride, int pad) {
    const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
    for (int nc = 0; nc < N * C; ++nc)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow) {
                float sum = 0.f;
                for (int kh = 0; kh < KH; ++kh)
                    for (int kw = 0; kw < KW; ++kw) {
                        const int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) sum += x[((size_t)nc * H + ih) * W + iw];
                    }
                y[((size_t)nc * Ho + oh) * Wo + ow] = sum / (float)(KH * KW);
            }
}

// cpu_backend.ixx:994-1023 — each output's gradient times 1/(KH*KW) added to its valid taps.
void omrefAvgPool2dBackward(const float* gO, float* gI, int N, int C, int H, int W, int Ho, int Wo, int KH, int KW,
                            int stride, int pad) {
    for (size_t i = 0; i < (size_t)N * C * H * W; ++i) gI[i] = 0.f;
    const float scale = 1.0f / (float)(KH * KW);
    for (int nc = 0; nc < N * C; ++nc)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow) {
                const float g = gO[((size_t)nc * Ho + oh) * Wo + ow] * scale;
                for (int kh = 0; kh < KH; ++kh)
                    for (int kw = 0; kw < KW; ++kw) {
                        const int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) gI[((size_t)nc * H + ih) * W + iw] += g;
                    }
            }
}

// cpu_backend.ixx:1467-1488 — region [floor(o*H/OH), floor((o+1)*H/OH)) per axis, mean.
void omrefAdaptiveAvgPool2d(const float* x, float* y, int N, int C, int H, int W, int OH, int OW) {
    for (int nc = 0; nc < N * C; ++nc)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow) {
                const int h0 = oh * H / OH, h1 = (oh + 1) * H / OH, w0 = ow * W / OW, w1 = (ow + 1) * W / OW;
                float sum = 0.f;
                int cnt = 0;
                for (int ih = h0; ih < h1; ++ih)
                    for (int iw = w0; iw < w1; ++iw) {
                        sum += x[((size_t)nc * H + ih) * W + iw];
                        ++cnt;
                    }
                y[((size_t)nc * OH + oh) * OW + ow] = sum / (float)cnt;
            }
}

// cpu_backend.ixx:1491-1510 — gradient / region size added over the region.
void omrefAdaptiveAvgPool2dBackward(const float* gO, float* gI, int N, int C, int H, int W, int OH, int OW) {
    for (size_t i = 0; i < (size_t)N * C * H * W; ++i) gI[i] = 0.f;
    for (int nc = 0; nc < N * C; ++nc)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow) {
                const int h0 = oh * H / OH, h1 = (oh + 1) * H / OH, w0 = ow * W / OW, w1 = (ow + 1) * W / OW;
                const float g = gO[((size_t)nc * OH + oh) * OW + ow] / (float)((h1 - h0) * (w1 - w0));
                for (int ih = h0; ih < h1; ++ih)
                    for (int iw = w0; iw < w1; ++iw) gI[((size_t)nc * H + ih) * W + iw] += g;
            }
}

// cpu_backend.ixx:352-370 — per row: max, exp(x - max), sequential sum, divide.
void omrefSoftmax(const float* in, float* out, int rows, int cols) {
    for (int b = 0; b < rows; ++b) {
        const float* r = in + (size_t)b * cols;
        float* o = out + (size_t)b * cols;
        float m = r[0];
        for (int j = 1; j < cols; ++j)
            if (r[j] > m) m = r[j];
        float sum = 0.f;
        for (int j = 0; j < cols; ++j) {
            o[j] = std::exp(r[j] - m);
            sum += o[j];
        }
        for (int j = 0; j < cols; ++j) o[j] /= sum;
    }
}

// cpu_backend.ixx:375-388 — loss -= log(max(p, 1e-7)) over the elements whose target
// exceeds 0.5, in (row, class) order; divided by the batch.
float omrefCrossEntropy(const float* pred, const float* tgt, int rows, int cols) {
    float loss = 0.f;
    for (int b = 0; b < rows; ++b)
        for (int j = 0; j < cols; ++j)
            if (tgt[(size_t)b * cols + j] > 0.5f) {
                float p = pred[(size_t)b * cols + j];
                if (p < 1e-7f) p = 1e-7f;
                loss -= std::log(p);
            }
    return loss / (float)rows;
}

// cpu_backend.ixx:393-410 — grad = (softmax - target) * (1 / batch).
void omrefCrossEntropySoftmaxBackward(const float* s, const float* t, float* g, int rows, int cols) {
    const float scale = 1.0f / (float)rows;
    const size_t n = (size_t)rows * cols;
    for (size_t i = 0; i < n; ++i) g[i] = (s[i] - t[i]) * scale;
}

// autograd.ixx:428-433 (AddBiasBackward, CPU path) — bias gradient: the zeroed
// gradient accumulates every row in order; for an [N, C, HW] gradient the
// rows are the (n, hw) pairs in that order.
void omrefAddBiasBackward(const float* g, float* gb, int N, int C, int HW) {
    for (int c = 0; c < C; ++c) gb[c] = 0.f;
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < C; ++c)
            for (int hw = 0; hw < HW; ++hw) gb[c] += g[((size_t)n * C + c) * HW + hw];
}

// om.engine.vit.ixx:193-236 (MultiHeadAttention::forward, CPU path, after the QKV
// projection): split heads with Q scaled, scores = Q x K^T (transpose2d +
// batchedMatmul), softmax over the last dim, context = P x V, merge heads.
// qkv [B*S, 3*H*D] -> out [B*S, H*D].
void omrefAttention(const float* qkv, float* out, int B, int S, int H, int D, float scale) {
    const int Dm = H * D, BH = B * H;
    std::vector<float> Q((size_t)BH * S * D), K((size_t)BH * S * D), V((size_t)BH * S * D);
    for (int n = 0; n < B; ++n)
        for (int s = 0; s < S; ++s) {
            const float* row = qkv + ((size_t)n * S + s) * 3 * Dm;
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    const size_t o = (((size_t)n * H + h) * S + s) * D + d;
                    Q[o] = row[h * D + d] * scale;
                    K[o] = row[Dm + h * D + d];
                    V[o] = row[2 * Dm + h * D + d];
                }
        }
    std::vector<float> kT((size_t)D * S), sc((size_t)S * S), P((size_t)S * S), ctx((size_t)S * D);
    for (int bh = 0; bh < BH; ++bh) {
        omrefTranspose2d(K.data() + (size_t)bh * S * D, kT.data(), S, D);
        omrefMatmul(Q.data() + (size_t)bh * S * D, kT.data(), sc.data(), S, D, S);
        omrefSoftmax(sc.data(), P.data(), S, S);
        omrefMatmul(P.data(), V.data() + (size_t)bh * S * D, ctx.data(), S, S, D);
        const int n = bh / H, h = bh % H;
        for (int s = 0; s < S; ++s)
            for (int d = 0; d < D; ++d) out[((size_t)n * S + s) * Dm + h * D + d] = ctx[(size_t)s * D + d];
    }
}

// cpu_backend.ixx:290-294 — CPUBackend::sum: one float accumulator, elements in order.
float omrefSum(const float* x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i];
    return s;
}

// vit.ixx:196-212 (MultiHeadAttention::forward, CPU branch) — qkv [B*S, 3*H*D] split into
// Q, K, V [B*H, S, D], Q multiplied by scale (the map omCudaQkvSplitHeads also uses).
void omrefQkvSplitHeads(const float* qkv, float* q, float* k, float* v, int B, int S, int H, int D, float scale) {
    const int Dm = H * D;
    for (int n = 0; n < B; ++n)
        for (int s = 0; s < S; ++s) {
            const float* row = qkv + ((size_t)n * S + s) * 3 * Dm;
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    const size_t o = (((size_t)n * H + h) * S + s) * D + d;
                    q[o] = row[h * D + d] * scale;
                    k[o] = row[Dm + h * D + d];
                    v[o] = row[2 * Dm + h * D + d];
                }
        }
}

// vit.ixx:220-232 — [B*H, S, D] merged back into [B*S, H*D].
void omrefMergeHeads(const float* in, float* out, int B, int S, int H, int D) {
    const int Dm = H * D;
    for (int n = 0; n < B; ++n)
        for (int s = 0; s < S; ++s)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d)
                    out[((size_t)n * S + s) * Dm + h * D + d] = in[(((size_t)n * H + h) * S + s) * D + d];
}

// cpu_backend.ixx:147-160, simd.ixx:180-200 — elementwise a + b.
void omrefAdd(const float* a, const float* b, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

// difference; the GPU path converts with round-to-nearest-even instead.
uint16_t omrefFloatToHalfTrunc(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 31) & 1u, ex = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    uint16_t he = 0, hm = 0;
    const int ne = (int)ex - 127 + 15;
    if (ex == 0xff) {
        he = 0x1f;
        if (man) { hm = (uint16_t)(man >> 13); if (!hm) hm = 1; }
    } else if (ex == 0) {
        he = 0; hm = 0;
    } else if (ne >= 0x1f) {
        he = 0x1f; hm = 0;
    } else if (ne <= 0) {
        if (ne >= -10) hm = (uint16_t)((man | 0x800000u) >> (14 - ne));
    } else {
        he = (uint16_t)ne;
        hm = (uint16_t)(man >> 13);
    }
    return (uint16_t)((sign << 15) | (he << 10) | hm);
}

void omrefFloatToHalfTruncN(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = omrefFloatToHalfTrunc(in[i]);
}

int omrefHasAvx2(void) {
#ifdef OMREF_AVX2
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

int omrefMaxThreads(void) { return omp_get_max_threads(); }

}  // extern "C"
