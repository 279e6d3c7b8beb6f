// unfused_chain.hip -- the five-kernel lowering of the chain (matmul, row max,
// exp, row sum, divide), the "baseline" side of the A/B harness.  Mirrors the
// reference's unfused lowering kernel by kernel
// (bench/baselines/default/baseline/04c.after_linalg_to_loops.mlir:37-124
// matmul, :129-186 max, :188-214 exp, :219-276 sum, :278-303 divide).  The
// matmul is chain_tile_kernel with the logits epilogue; the four row kernels
// are below.  One workgroup per row, logits in f32 in the workspace.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tile_layout.h"
#include "wtc_kernels.h"

namespace wtc {

template <typename Op>
__device__ inline float block_reduce(float x, Op op, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = op(x, __shfl_xor(x, off));
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = x;
  __syncthreads();
  x = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) x = op(x, red[i]);
  __syncthreads();
  return x;
}

struct MaxOp { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct SumOp { __device__ float operator()(float a, float b) const { return a + b; } };

// max[r] = max_j C[r, j], from -FLT_MAX as the chain's fill
// (mlir/matmul_softmax_chain.mlir max init).
__global__ void __launch_bounds__(256) rowmax_kernel(const float* __restrict__ C,
                                                     float* __restrict__ mx, int64_t N) {
  __shared__ float red[4];
  const float* row = C + (int64_t)blockIdx.x * N;
  float m = -3.4028235e38f;
  for (int64_t j = threadIdx.x; j < N; j += blockDim.x) m = fmaxf(m, row[j]);
  m = block_reduce(m, MaxOp(), red);
  if (threadIdx.x == 0) mx[blockIdx.x] = m;
}

// C[r, j] = exp(C[r, j] - max[r]), in place.
__global__ void __launch_bounds__(256) expsub_kernel(float* __restrict__ C,
                                                     const float* __restrict__ mx, int64_t N) {
  float* row = C + (int64_t)blockIdx.x * N;
  const float m = mx[blockIdx.x];
  for (int64_t j = threadIdx.x; j < N; j += blockDim.x) row[j] = expf(row[j] - m);
}

// sum[r] = sum_j E[r, j], from 0.
__global__ void __launch_bounds__(256) rowsum_kernel(const float* __restrict__ E,
                                                     float* __restrict__ sm, int64_t N) {
  __shared__ float red[4];
  const float* row = E + (int64_t)blockIdx.x * N;
  float s = 0.0f;
  for (int64_t j = threadIdx.x; j < N; j += blockDim.x) s += row[j];
  s = block_reduce(s, SumOp(), red);
  if (threadIdx.x == 0) sm[blockIdx.x] = s;
}

// out[r, j] = E[r, j] / sum[r], converted to the output type.
template <int OUT_DT>
__global__ void __launch_bounds__(256) rowdiv_kernel(const float* __restrict__ E,
                                                     const float* __restrict__ sm,
                                                     void* __restrict__ out, int64_t N) {
  const int64_t r = blockIdx.x;
  const float* row = E + r * N;
  const float s = sm[r];
  for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
    const float y = row[j] / s;
    if constexpr (OUT_DT == DT_F32) {
      static_cast<float*>(out)[r * N + j] = y;
    } else if constexpr (OUT_DT == DT_F16) {
      static_cast<_Float16*>(out)[r * N + j] = (_Float16)y;
    } else {
      static_cast<__bf16*>(out)[r * N + j] = (__bf16)y;
    }
  }
}

const void* rowmax_kernel_symbol() { return reinterpret_cast<const void*>(&rowmax_kernel); }
const void* expsub_kernel_symbol() { return reinterpret_cast<const void*>(&expsub_kernel); }
const void* rowsum_kernel_symbol() { return reinterpret_cast<const void*>(&rowsum_kernel); }
const void* rowdiv_kernel_symbol(int out_dt) {
  switch (out_dt) {
    case DT_F32: return reinterpret_cast<const void*>(&rowdiv_kernel<DT_F32>);
    case DT_F16: return reinterpret_cast<const void*>(&rowdiv_kernel<DT_F16>);
    case DT_BF16: return reinterpret_cast<const void*>(&rowdiv_kernel<DT_BF16>);
  }
  return nullptr;
}

}  // namespace wtc
