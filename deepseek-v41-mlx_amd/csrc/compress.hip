// Softmax-gated KV pooling of the compressor (ratio > 1), deepseek_v41_mlx/compressor.py:58-79.
//
// One workgroup per (batch row, complete group). A thread owns channels; the pooling softmax is
// per channel over the ratio axis, so only the RMSNorm of the pooled vector crosses threads.
// The carried partial group lives in kv_state/score_state [bsz, ratio, dim] (fp32). Only the
// group-0 workgroup reads the carried rows, and it rewrites the state after reading it, in the
// same thread per channel, so no other workgroup races with the update.
#include "common.h"

namespace dsv41 {

constexpr int kPoolThreads = 256;
constexpr int kPoolMaxCh = 4;  // dim <= 1024

template <typename T>
__global__ __launch_bounds__(kPoolThreads) void compress_pool_kernel(
    const float* __restrict__ kv, const float* __restrict__ score, float* kv_state, float* score_state,
    T* latents, const float* __restrict__ norm_w, int n, int dim, int ratio, int m, int g, int rem, float eps) {
  __shared__ float red[kPoolThreads / 64];
  const int b = blockIdx.y;
  const int j = blockIdx.x;
  const float* kvb = kv + (int64_t)b * n * dim;
  const float* scb = score + (int64_t)b * n * dim;
  float* kst = kv_state + (int64_t)b * ratio * dim;
  float* sst = score_state + (int64_t)b * ratio * dim;

  if (g > 0) {
    float pooled[kPoolMaxCh];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kPoolMaxCh; ++u) {
      const int c = threadIdx.x + u * kPoolThreads;
      pooled[u] = 0.0f;
      if (c >= dim) continue;
      // rows j*ratio .. j*ratio+ratio-1 of concat(state[:m], chunk)
      float mx = -INFINITY;
      for (int q = 0; q < ratio; ++q) {
        const int t = j * ratio + q;
        const float sc = t < m ? sst[(int64_t)t * dim + c] : scb[(int64_t)(t - m) * dim + c];
        mx = fmaxf(mx, sc);
      }
      float den = 0.0f;
      for (int q = 0; q < ratio; ++q) {
        const int t = j * ratio + q;
        const float sc = t < m ? sst[(int64_t)t * dim + c] : scb[(int64_t)(t - m) * dim + c];
        den += expf(sc - mx);
      }
      float acc = 0.0f;
      for (int q = 0; q < ratio; ++q) {
        const int t = j * ratio + q;
        const float sc = t < m ? sst[(int64_t)t * dim + c] : scb[(int64_t)(t - m) * dim + c];
        const float v = t < m ? kst[(int64_t)t * dim + c] : kvb[(int64_t)(t - m) * dim + c];
        acc += v * (expf(sc - mx) / den);
      }
      pooled[u] = io<T>::rnd(acc);  // pooled.astype(dtype) before the norm
      ss += pooled[u] * pooled[u];
    }
    ss = group_sum(ss, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kPoolThreads / 64; ++w) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
    T* out = latents + ((int64_t)b * g + j) * dim;
#pragma unroll
    for (int u = 0; u < kPoolMaxCh; ++u) {
      const int c = threadIdx.x + u * kPoolThreads;
      if (c < dim) io<T>::st(out + c, norm_w[c] * (pooled[u] * inv));
    }
  }

  // carry-out of the open group (compressor.py:70-73), by the group-0 workgroup only
  if (j == 0 && rem > 0) {
    const int total = m + n;
    for (int u = 0; u < kPoolMaxCh; ++u) {
      const int c = threadIdx.x + u * kPoolThreads;
      if (c >= dim) continue;
      for (int r = 0; r < rem; ++r) {
        const int t = total - rem + r;       // concat row
        if (t < m) continue;                 // carried row already in place (t == r here)
        kst[(int64_t)r * dim + c] = kvb[(int64_t)(t - m) * dim + c];
        sst[(int64_t)r * dim + c] = scb[(int64_t)(t - m) * dim + c];
      }
    }
  }
}

}  // namespace dsv41

using namespace dsv41;

extern "C" int dsv41_compress_pool(const float* kv, const float* score, float* kv_state, float* score_state,
                                   void* latents, const float* norm_w, int32_t bsz, int32_t n, int32_t dim,
                                   int32_t ratio, int32_t start_pos, float eps, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_compress_pool";
  DSV41_REQUIRE(kv && score && kv_state && score_state && norm_w, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(ratio > 1, DSV41_E_ARG, "%s: ratio %d must be > 1 (ratio 1 has no pooling)", what, ratio);
  DSV41_REQUIRE(dim > 0 && dim <= kPoolThreads * kPoolMaxCh, DSV41_E_SHAPE, "%s: dim %d > %d", what, dim,
                kPoolThreads * kPoolMaxCh);
  const int m = start_pos % ratio;
  const int total = m + n;
  const int g = total / ratio;
  const int rem = total % ratio;
  DSV41_REQUIRE(g == 0 || latents, DSV41_E_ARG, "%s: latents is null but %d groups complete", what, g);
  if (bsz == 0 || (g == 0 && rem == 0)) return 0;
  DSV41_REQUIRE(bsz < 65536, DSV41_E_ARG, "%s: bsz too large", what);
  dim3 grid((unsigned)(g > 0 ? g : 1), (unsigned)bsz);
  if (dtype == DSV41_F32)
    hipLaunchKernelGGL(compress_pool_kernel<float>, grid, dim3(kPoolThreads), 0, stream, kv, score, kv_state,
                       score_state, (float*)latents, norm_w, n, dim, ratio, m, g, rem, eps);
  else if (dtype == DSV41_BF16)
    hipLaunchKernelGGL(compress_pool_kernel<bf16_t>, grid, dim3(kPoolThreads), 0, stream, kv, score, kv_state,
                       score_state, (bf16_t*)latents, norm_w, n, dim, ratio, m, g, rem, eps);
  else
    return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  return check_launch(what);
}
