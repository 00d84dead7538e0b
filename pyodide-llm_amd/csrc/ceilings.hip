// ceilings.hip — loops of one kind of work only, for the ceilings the engine's kernels are measured against
// (kernels/ceilings.ts, kernels/ceilings_relaxed.ts on the device):
//   read: the memory's streaming read rate, over a few launch shapes (ceilings.ts:9-25 read());
//   valu: float32 multiply + add pairs on registers, each rounded (no FMA, no packed FP32): the form of every ordered
//     float32 step of the exact path (ceilings.ts:27-50 fma());
//   mfma: v_mfma_i32_32x32x32_i8 on registers, the prompt GEMM's instruction at its own rate (the device's form of
//     ceilings_relaxed.ts:33-50 dotRegisters()).
// Each loop returns a checksum of everything it computed, which the caller can compute too: a loop the compiler cut
// short returns another number.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// a wave reads tiles of 64 L uint4 (L loads of 16 bytes a lane, all issued before the first is used), tile w + waves
// * k for wave w of the launch; the words added lane by lane (uint32, wrapping, order-free) into the block's four
// partial sums, partial[4 * block + j] (no atomics: a few addresses taken by every block would serialize the launch).
// A load past the end is clamped to the buffer's last 16 bytes and adds nothing.
template <int L>
__global__ __launch_bounds__(256) void read_ceiling_kernel(const uint4 *p, int64_t n16, uint32_t *partial) {
  __shared__ uint4 waves[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nw = (int64_t)gridDim.x * 4, tiles = (n16 + 64 * L - 1) / (64 * L);
  uint4 acc = {0u, 0u, 0u, 0u};
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave; t < tiles; t += nw) {
    uint4 v[L];
#pragma unroll
    for (int u = 0; u < L; ++u) v[u] = p[min(t * 64 * L + u * 64 + lane, n16 - 1)];
#pragma unroll
    for (int u = 0; u < L; ++u) {
      if (t * 64 * L + u * 64 + lane < n16) {
        acc.x += v[u].x;
        acc.y += v[u].y;
        acc.z += v[u].z;
        acc.w += v[u].w;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    acc.x += __shfl_xor(acc.x, o, 64);
    acc.y += __shfl_xor(acc.y, o, 64);
    acc.z += __shfl_xor(acc.z, o, 64);
    acc.w += __shfl_xor(acc.w, o, 64);
  }
  if (lane == 0) waves[wave] = acc;
  __syncthreads();
  if (threadIdx.x < 4) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(waves);
    partial[4 * blockIdx.x + threadIdx.x] = w[threadIdx.x] + w[4 + threadIdx.x] + w[8 + threadIdx.x] + w[12 + threadIdx.x];
  }
}

// the launch shapes the read ceiling is taken over (loads a lane per tile, blocks of 256 threads at most)
struct ReadShape {
  int loads, blocks;
};
constexpr ReadShape READ_SHAPES[] = {{8, 256}, {8, 512}, {4, 512}, {8, 1024}, {16, 1024}, {16, 2048}};
constexpr int READ_SHAPE_COUNT = sizeof(READ_SHAPES) / sizeof(READ_SHAPES[0]);

// ceilings.ts fma() for one lane: w0..w3 = w + {0, 2^-10, 2^-9, 3 * 2^-10}, x = x0, y = x0 + 0.25, accumulators 0..7;
// a pass adds w_j * x (j = 0..3) and w_j * y to the eight (a multiply and an add each, both rounded), then x -= step,
// y -= step. Lane l starts x and y at + spread * l (spread 0: every lane computes the same; a value the compiler cannot
// see, so that it keeps the work per lane). Lane 0 of each wave writes ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 +
// a7)) to out[wave]; ceilings.ts fma() returns the sum of its four equal lanes of that value.
__global__ __launch_bounds__(256) void valu_ceiling_kernel(int32_t passes, float w, float x0, float step, float spread,
                                                           float *out) {
  const float shift = spread * (float)(threadIdx.x & 63);
  const float w0 = w, w1 = w + 0.0009765625f, w2 = w + 0.001953125f, w3 = w + 0.0029296875f;
  float x = x0 + shift, y = (x0 + 0.25f) + shift;
  float a0 = 0.f, a1 = 1.f, a2 = 2.f, a3 = 3.f, a4 = 4.f, a5 = 5.f, a6 = 6.f, a7 = 7.f;
#pragma unroll 4
  for (int32_t i = 0; i < passes; ++i) {
    a0 = a0 + w0 * x;
    a1 = a1 + w1 * x;
    a2 = a2 + w2 * x;
    a3 = a3 + w3 * x;
    a4 = a4 + w0 * y;
    a5 = a5 + w1 * y;
    a6 = a6 + w2 * y;
    a7 = a7 + w3 * y;
    x = x - step;
    y = y - step;
  }
  const float s = ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7));
  if ((threadIdx.x & 63) == 0) out[((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6] = s;
}

constexpr int VALU_BLOCKS = 2048;  // 8 blocks of 4 waves a CU: 8 waves a SIMD, 8 chains each
constexpr int MFMA_BLOCKS = 1024;  // 4 waves a SIMD, 4 accumulators each

// dotRegisters on the matrix core: four 32x32 int32 accumulators, a pass one v_mfma_i32_32x32x32_i8 into each with
// every byte of A = first, flipped by flip (xor) after each pass, and every byte of B = times; accumulator n starts at
// 1000 n + e in its element e (every lane). Lane 0 of each wave writes the wave's sum (mod 2^32) of every element of
// the four accumulators to out[wave].
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int32_t passes, int32_t first, int32_t times, int32_t flip,
                                                           uint32_t *out) {
  const int32_t fb = (int32_t)((uint32_t)(uint8_t)first * 0x01010101u);
  const int32_t tb = (int32_t)((uint32_t)(uint8_t)times * 0x01010101u);
  const int32_t xb = (int32_t)((uint32_t)(uint8_t)flip * 0x01010101u);
  v4i a = {fb, fb, fb, fb};
  const v4i b = {tb, tb, tb, tb}, f = {xb, xb, xb, xb};
  v16i c0, c1, c2, c3;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    c0[e] = e;
    c1[e] = 1000 + e;
    c2[e] = 2000 + e;
    c3[e] = 3000 + e;
  }
  for (int32_t i = 0; i < passes; ++i) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    a ^= f;
  }
  uint32_t s = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += (uint32_t)c0[e] + (uint32_t)c1[e] + (uint32_t)c2[e] + (uint32_t)c3[e];
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) out[((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6] = s;
}

}  // namespace

int32_t read_ceiling_shapes() { return READ_SHAPE_COUNT; }

int32_t read_ceiling_blocks(int64_t bytes, int32_t shape) {
  const ReadShape rs = READ_SHAPES[shape];
  const int64_t tiles = (bytes / 16 + 64 * rs.loads - 1) / (64 * rs.loads);
  return (int32_t)std::min<int64_t>(rs.blocks, std::max<int64_t>(1, (tiles + 3) / 4));
}

int32_t read_ceiling_loads(int32_t shape) { return READ_SHAPES[shape].loads; }

hipError_t launch_read_ceiling(const void *p, int64_t bytes, int32_t shape, uint32_t *partial, hipStream_t s) {
  const dim3 grid(read_ceiling_blocks(bytes, shape));
  const uint4 *q = reinterpret_cast<const uint4 *>(p);
  switch (READ_SHAPES[shape].loads) {
    case 4: hipLaunchKernelGGL(read_ceiling_kernel<4>, grid, dim3(256), 0, s, q, bytes / 16, partial); break;
    case 8: hipLaunchKernelGGL(read_ceiling_kernel<8>, grid, dim3(256), 0, s, q, bytes / 16, partial); break;
    default: hipLaunchKernelGGL(read_ceiling_kernel<16>, grid, dim3(256), 0, s, q, bytes / 16, partial); break;
  }
  return hipGetLastError();
}

int32_t valu_ceiling_waves() { return VALU_BLOCKS * 4; }

hipError_t launch_valu_ceiling(int32_t passes, float w, float x0, float step, float spread, float *out,
                               hipStream_t s) {
  hipLaunchKernelGGL(valu_ceiling_kernel, dim3(VALU_BLOCKS), dim3(256), 0, s, passes, w, x0, step, spread, out);
  return hipGetLastError();
}

int32_t mfma_ceiling_waves() { return MFMA_BLOCKS * 4; }

hipError_t launch_mfma_ceiling(int32_t passes, int32_t first, int32_t times, int32_t flip, uint32_t *out,
                               hipStream_t s) {
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(MFMA_BLOCKS), dim3(256), 0, s, passes, first, times, flip, out);
  return hipGetLastError();
}

}  // namespace ple
