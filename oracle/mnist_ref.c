/* Test infrastructure only (the parity oracle; never linked into the product).
 *
 * Portable C restatement of the reference CPU GEMM used by the MNIST MLP path:
 * gemm_bias_relu_f32_cpu / gemm_bias_f32_cpu (lariaus/lokinfer kernels/cpu/gemm.cpp:44-113).
 * Per output element the reference accumulates c = fma(a[i, p], b[p, j], c) for p = 0 .. K-1 in order
 * (tile16 / tailColumns' vector path, gemm.cpp:44-66), then adds the bias, then applies max(., 0).
 * Compiled with -ffp-contract=off so the only fused operations are the explicit fmaf calls.
 */
#include <math.h>
#include <stdint.h>

void lk_ref_gemm_bias_act_f32(const float* a, const float* b, const float* bias, float* out, int64_t m, int64_t n,
                              int64_t k, int relu) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float c = 0.0f;
      for (int64_t p = 0; p < k; ++p) c = fmaf(a[i * k + p], b[p * n + j], c);
      if (bias) c = c + bias[j];
      if (relu) c = c > 0.0f ? c : 0.0f;
      out[i * n + j] = c;
    }
}

/* MNIST MLP forward (784 -> 128 ReLU -> [64 ReLU ->] 10): h = relu(x W1 + b1) ...; returns logits. */
void lk_ref_mlp_f32(const float* x, int64_t batch, const float* const* ws, const float* const* bs, const int64_t* dims,
                    int nlayers, float* scratch, float* out) {
  const float* in = x;
  float* bufs[2] = {scratch, scratch + batch * 4096};
  for (int l = 0; l < nlayers; ++l) {
    float* dst = l == nlayers - 1 ? out : bufs[l & 1];
    lk_ref_gemm_bias_act_f32(in, ws[l], bs[l], dst, batch, dims[l + 1], dims[l], l < nlayers - 1);
    in = dst;
  }
}
