// gnf4_floor.hip -- measurement kernels for bench.py (libgnf4_floor.so), not
// part of the operator library.
//
// They bound what a decode launch of the grouped 4-bit GEMM can reach on
// this GPU, measured the same way as the decode kernels (a graph of
// back-to-back launches):
//   k_floor_empty   a launch that does nothing: the per-launch cost of a
//                   dependent kernel in a graph (dispatch, the end-of-kernel
//                   cache write-back, the start of the next one).
//   k_floor_read    a plain read of exactly the bytes a decode launch reads
//                   (the packed [N, K/2] stack of every active expert), 16
//                   bytes per lane, each workgroup a contiguous 8 KiB of one
//                   expert's stack, one expert id per grid row read from a
//                   device table as the decode kernels do. Nothing is
//                   computed: the bytes are folded into an XOR that is stored
//                   only if it matches a constant, so the loads cannot be
//                   dropped. Of the geometries measured on MI355X (1..16
//                   loads per lane, 256..512 threads, the decode kernels'
//                   16-row tile pattern), one load per lane in 512-thread
//                   workgroups was the fastest.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;

__global__ void k_floor_empty() {}

__global__ void __launch_bounds__(512) k_floor_read(const uint8_t* __restrict__ B, int64_t sbe,
                                                    int64_t region, const int32_t* __restrict__ eids,
                                                    unsigned* __restrict__ sink) {
  const int64_t e = eids[blockIdx.y];
  const int64_t off = ((int64_t)blockIdx.x * 512 + threadIdx.x) * 16;
  const int n = region < 0x7FFFFFFF ? (int)region : 0x7FFFFFFF;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B + e * sbe), 0, n, 0x00020000);
  // bounds-checked load: lanes past the region read zeros
  const u32x4_t v = __builtin_bit_cast(
      u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off < region ? (int)off : n, 0, 0));
  const unsigned x = v[0] ^ v[1] ^ v[2] ^ v[3];
  if (x == 0x9E3779B9u) sink[0] = x;
}

}  // namespace

extern "C" {

// A graph-capturable empty launch of grid (gx, gy) x 512 threads.
int gnf4_floor_empty(int gx, int gy, void* stream) {
  if (gx <= 0 || gy <= 0) return -1;
  hipLaunchKernelGGL(k_floor_empty, dim3(gx, gy), dim3(512), 0, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Read region bytes of the stacks of experts eids[0..G) (stack e at
// B + e * sbe); sink: one device u32, written only by chance.
int gnf4_floor_read(const uint8_t* B, int64_t sbe, int64_t region, const int32_t* eids, int G,
                    void* sink, void* stream) {
  if (!B || !eids || !sink || G <= 0 || G > 65535 || region <= 0 || region > 0x7FFFFFFF)
    return -1;
  const int64_t gx = (region + 512 * 16 - 1) / (512 * 16);
  hipLaunchKernelGGL(k_floor_read, dim3((unsigned)gx, (unsigned)G), dim3(512), 0,
                     (hipStream_t)stream, B, sbe, region, eids, (unsigned*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
