/*
 * Brute-force float64 modulated deformable convolution (DCNv2), one offset
 * group.  TEST INFRASTRUCTURE ONLY: it pins oracle/kadconv_oracle.py's
 * vectorised deform_conv2d on small inputs and is never linked into the
 * product library.
 *
 * Semantics restate torchvision.ops.deform_conv2d as the reference itself
 * describes it (KAD-Conv/kadconv/acceleration/kadc_dcn_direct.py:57-107 and
 * kadc_dcn16_kernel.cu:206-266): for output (oy, ox) and tap k = ky*KW + kx,
 *   py = oy*stride - pad + ky*dil + offset[2k],  px = ox*stride - pad + kx*dil + offset[2k+1]
 * a sample is 0 when py <= -1, py >= H, px <= -1 or px >= W; otherwise the
 * four corners around floor() are blended and corners outside the image
 * contribute 0.  Layouts are NCHW; offset [N, 2K, Ho, Wo]; mask [N, K, Ho, Wo]
 * (mask may be NULL = all ones); weight [Co, Ci, KH, KW]; bias may be NULL.
 */
#include <math.h>
#include <stddef.h>

static double sample(const double *img, int H, int W, double py, double px) {
    if (py <= -1.0 || py >= H || px <= -1.0 || px >= W) return 0.0;
    double fy = floor(py), fx = floor(px);
    int y0 = (int)fy, x0 = (int)fx, y1 = y0 + 1, x1 = x0 + 1;
    double ly = py - fy, lx = px - fx, hy = 1.0 - ly, hx = 1.0 - lx;
    double v00 = (y0 >= 0 && x0 >= 0) ? img[(size_t)y0 * W + x0] : 0.0;
    double v01 = (y0 >= 0 && x1 <= W - 1) ? img[(size_t)y0 * W + x1] : 0.0;
    double v10 = (y1 <= H - 1 && x0 >= 0) ? img[(size_t)y1 * W + x0] : 0.0;
    double v11 = (y1 <= H - 1 && x1 <= W - 1) ? img[(size_t)y1 * W + x1] : 0.0;
    return hy * hx * v00 + hy * lx * v01 + ly * hx * v10 + ly * lx * v11;
}

int oracle_dcn_brute_f64(const double *x, const double *offset, const double *mask,
                         const double *weight, const double *bias, double *out,
                         int N, int Ci, int H, int W, int Co, int KH, int KW,
                         int stride, int pad, int dil) {
    int Ho = (H + 2 * pad - dil * (KH - 1) - 1) / stride + 1;
    int Wo = (W + 2 * pad - dil * (KW - 1) - 1) / stride + 1;
    int K = KH * KW;
    if (Ho <= 0 || Wo <= 0) return -1;
    size_t plane = (size_t)Ho * Wo;
    for (int n = 0; n < N; ++n)
        for (int co = 0; co < Co; ++co)
            for (int oy = 0; oy < Ho; ++oy)
                for (int ox = 0; ox < Wo; ++ox) {
                    double acc = bias ? bias[co] : 0.0;
                    size_t p = (size_t)oy * Wo + ox;
                    for (int ci = 0; ci < Ci; ++ci) {
                        const double *img = x + ((size_t)n * Ci + ci) * H * W;
                        for (int k = 0; k < K; ++k) {
                            int ky = k / KW, kx = k % KW;
                            double dy = offset[((size_t)n * 2 * K + 2 * k) * plane + p];
                            double dx = offset[((size_t)n * 2 * K + 2 * k + 1) * plane + p];
                            double m = mask ? mask[((size_t)n * K + k) * plane + p] : 1.0;
                            double py = (double)(oy * stride - pad + ky * dil) + dy;
                            double px = (double)(ox * stride - pad + kx * dil) + dx;
                            double w = weight[(((size_t)co * Ci + ci) * KH + ky) * KW + kx];
                            acc += w * m * sample(img, H, W, py, px);
                        }
                    }
                    out[((size_t)n * Co + co) * plane + p] = acc;
                }
    return 0;
}
