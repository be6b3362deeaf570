// Floors the sampler kernels are measured against, under rocprofv3 --kernel-trace (profiles/launch_floor.md):
//   - empty_kernel on the sampler's grid shapes: what a launch costs with no work (a kernel's duration includes
//     its workgroups' dispatch and retirement);
//   - read_floor: a pure streaming read of B rows of V fp32 with the small-k kernel's load pattern (256 threads, 16
//     nontemporal float4 loads each, all issued at once) and nothing else but a maximum per workgroup: the time the
//     bytes take to arrive, for the headline batch (B=64, V=262144) and for config 1's row (B=1, V=65536, 4 loads).
// usage: launch_floor [launches]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

__global__ __launch_bounds__(512) void empty_kernel(int* out) {
    if (out && threadIdx.x == 0 && blockIdx.x == 0xFFFFFFFFu) *out = 1;    // never taken: keeps the argument alive
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ f32x4 raw_load(__amdgpu_buffer_rsrc_t rs, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");

template <int NL>
__global__ __launch_bounds__(256) void read_floor(const float* x, int V, int nseg, float* out) {
    constexpr int SEG = 256 * NL * 4;
    const int i = blockIdx.x, xc = i % 8, j = i / 8;
    const int row = xc + 8 * (j / nseg), seg = j % nseg;
    const float* p = x + (long)row * V + (long)seg * SEG;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, SEG * 4,
                                                                        0x00020000);
    f32x4 v[NL];
#pragma unroll
    for (int q = 0; q < NL; ++q) v[q] = raw_load(rs, (q * 256 + (int)threadIdx.x) * 16, 0, 2);
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < NL; ++q) m = fmaxf(m, fmaxf(fmaxf(v[q].x, v[q].y), fmaxf(v[q].z, v[q].w)));
    if (threadIdx.x % 64 == 0 || m > 3e38f) out[i * 4 + threadIdx.x / 64] = m;
}

#define CK(x) do { if ((x) != hipSuccess) { fprintf(stderr, "HIP error at %d\n", __LINE__); return 1; } } while (0)

int main(int argc, char** argv) {
    const int n = argc > 1 ? atoi(argv[1]) : 200;
    float* x = nullptr;
    float* out = nullptr;
    const size_t copies = 8, rowbytes = (size_t)64 * 262144 * 4;           // rotated past the 256 MB MALL
    CK(hipMalloc(&x, copies * rowbytes));
    CK(hipMemset(x, 0, copies * rowbytes));
    CK(hipMalloc(&out, 1 << 20));
    const unsigned shapes[][2] = {{16, 256}, {1024, 256}, {576, 512}, {4096, 256}};
    for (const auto& sh : shapes)
        for (int i = 0; i < n; ++i) hipLaunchKernelGGL(empty_kernel, dim3(sh[0]), dim3(sh[1]), 0, 0, (int*)out);
    for (int i = 0; i < n; ++i)                                             // headline: 64 x 262144, 1024 workgroups
        hipLaunchKernelGGL(read_floor<16>, dim3(1024), dim3(256), 0, 0,
                           x + (i % copies) * (rowbytes / 4), 262144, 16, out);
    for (int i = 0; i < n; ++i)                                             // config 1: 1 x 65536, 16 workgroups
        hipLaunchKernelGGL(read_floor<4>, dim3(8 * 16), dim3(256), 0, 0, x + (i % copies) * (rowbytes / 4), 65536,
                           16, out);
    CK(hipDeviceSynchronize());
    printf("launch_floor: %d launches of each shape\n", n);
    return 0;
}
