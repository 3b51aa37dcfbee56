// floor_probe.hip — the speed-of-light reference for the 8B decode sweep.
//
// Not part of libspq4k. Replays, as one HIP graph, the same sequence of 145
// dependent launches as bench.py's decode8b step (36 x [q/k/v 14.16 MB, o
// 9.44 MB, gate/up 56.62 MB, down 28.31 MB] + lm_head 350.06 MB over 4.26 GB
// of distinct buffers) with a kernel that only streams the bytes (no compute,
// no activations), and times an empty kernel launched 145 times the same way.
// The first is the best a per-op decode sweep can do on this GPU; the second
// is the fixed cost of one dependent launch.
//
//   ./floor_probe            (built by `make -C shannon-prime-burnhard_amd`)
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <vector>

#define CK(x)                                                                            \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess) {                                                          \
            fprintf(stderr, "%s: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__);  \
            exit(1);                                                                     \
        }                                                                                \
    } while (0)

__global__ void empty_kernel(int* p) {
    if (threadIdx.x == 1000) p[0] = 1;
}

// grid-stride read of n16 16-byte words, U loads in flight per lane
template <int U>
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ src, size_t n16, unsigned* out) {
    const size_t stride = (size_t)gridDim.x * 256 * U;
    unsigned a = 0;
    for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n16; base += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = base + (size_t)u * 256;
            v[u] = src[i < n16 ? i : n16 - 1];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) a ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (a == 0x12345678u) out[blockIdx.x] = a;   // keeps the loads; never true for the fill below
}

struct Launch {
    const uint4* p;
    size_t bytes;
};

static float replay(hipStream_t s, const std::vector<Launch>& seq, int grid, unsigned* out, int reps) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    for (const Launch& l : seq) {
        if (l.p)
            hipLaunchKernelGGL((read_kernel<4>), dim3(grid), dim3(256), 0, s, l.p, l.bytes / 16, out);
        else
            hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s, (int*)out);
    }
    CK(hipStreamEndCapture(s, &g));
    CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CK(hipGraphLaunch(ge, s));
    CK(hipStreamSynchronize(s));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a, s));
    for (int r = 0; r < reps; ++r) CK(hipGraphLaunch(ge, s));
    CK(hipEventRecord(b, s));
    CK(hipEventSynchronize(b));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, a, b));
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
    CK(hipGraphExecDestroy(ge));
    CK(hipGraphDestroy(g));
    return ms / reps;
}

int main() {
    hipStream_t s;
    CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    unsigned* out;
    CK(hipMalloc(&out, 1 << 20));
    const size_t qkv = 6144ull * 2304, o = 4096ull * 2304, gu = 24576ull * 2304, dn = 4096ull * 6912,
                 lm = 151936ull * 2304;
    const size_t step = (qkv + o + gu + dn) * 36 + lm;
    uint8_t* pool;
    CK(hipMalloc(&pool, step));
    CK(hipMemset(pool, 1, step));
    CK(hipDeviceSynchronize());

    std::vector<Launch> empty(145, Launch{nullptr, 0});
    const float e_ms = replay(s, empty, 0, out, 50);
    printf("empty kernel, 145 dependent launches in one graph: %.3f us per launch\n", e_ms * 1e3 / 145);

    std::vector<Launch> seq;
    size_t off = 0;
    for (int L = 0; L < 36; ++L)
        for (size_t b : {qkv, o, gu, dn}) {
            seq.push_back({(const uint4*)(pool + off), b});
            off += b;
        }
    seq.push_back({(const uint4*)(pool + off), lm});
    for (int grid : {512, 1024}) {
        const float ms = replay(s, seq, grid, out, 20);
        printf("streaming read, 8B decode sweep (%zu B in 145 launches, grid %d x 256, 4 x 16 B in flight per lane): "
               "%.1f us per step = %.1f GB/s = %.1f%% of 8 TB/s\n",
               step, grid, ms * 1e3, step / (ms * 1e-3) / 1e9, step / (ms * 1e-3) / 8e10);
    }
    printf("per launch size (grid 1024, cold, %s):\n", "distinct buffers");
    for (size_t b : {o, qkv, dn, gu, lm}) {
        std::vector<Launch> sq;
        size_t n = step / b;
        if (n > 60) n = 60;
        for (size_t i = 0; i < n; ++i) sq.push_back({(const uint4*)(pool + i * b), b});
        const float ms = replay(s, sq, 1024, out, 5);
        printf("  %8.2f MB: %.2f us per launch, %.1f GB/s\n", b / 1e6, ms * 1e3 / n, b * n / (ms * 1e-3) / 1e9);
    }
    CK(hipFree(pool));
    CK(hipFree(out));
    return 0;
}
