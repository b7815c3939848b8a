// calibrate.hip -- measures the machine constants the MI355X launch model
// needs and that no data sheet gives: the cost of one launch in a stream of
// back-to-back launches and inside a captured graph, the latency of a
// dependent global load (idle and with every CU loading, from HBM and from
// L2), the bandwidth of a plain HBM copy, the rate at which one CU reads
// L2-resident data, the LDS read rate for the record strides the kernels
// use, and the shader clock.
//
// Every kernel here is bounded: the pointer chases follow a single cycle over
// an index array whose entries are all in range, with a fixed hop count; the
// copies and reads use grid-stride loops over their own buffers.
//
// Output: one JSON line on stdout.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <numeric>
#include <random>
#include <vector>

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      return 1;                                                                        \
    }                                                                                  \
  } while (0)

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStride = 64;  // int32 slots between chased entries (256 bytes)

__global__ void empty_kernel(int *p) {
  if (p && threadIdx.x == 1024) p[0] = 0;  // never taken: keeps the argument live
}

// Every lane follows the cycle `hops` times from its own entry (so the loads
// are per-lane vector loads); entry i of the cycle lives at next[i * kStride].
__global__ void chase_kernel(const int *__restrict__ next, int hops, int n, int *out) {
  const unsigned g = blockIdx.x * blockDim.x + threadIdx.x;
  int j = (int)((g * 2654435761u) % (unsigned)n);
  for (int h = 0; h < hops; ++h) j = next[(size_t)j * kStride];
  if (j == -1) out[g] = j;  // never true: keeps the chase live
}

// Grid-stride copy, four independent 16-byte loads per lane per step; n is a
// multiple of 4 x the grid's lane count.
__global__ void copy_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, size_t n) {
  const size_t lanes = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += 4 * lanes) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = src[i + u * lanes];
#pragma unroll
    for (int u = 0; u < 4; ++u) dst[i + u * lanes] = v[u];
  }
}

// Streaming kernels for the attainable HBM rate: grid-stride over n 16-byte
// elements, U independent 16-byte accesses per lane in flight, every access
// bounds-checked, non-temporal (streaming) loads and stores.  The read kernel
// folds what it loads into one value per lane and stores it only when it
// equals a value no finite input produces, so the loads are kept without
// adding traffic.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ void stream_read_kernel(const f32x4 *__restrict__ src, size_t n, float *out) {
  const size_t lanes = (size_t)gridDim.x * blockDim.x;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += U * lanes) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (i + u * lanes < n) v[u] = __builtin_nontemporal_load(&src[i + u * lanes]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u];
  }
  const float t = acc.x + acc.y + acc.z + acc.w;
  if (t == -1.f) out[blockIdx.x] = t;
}

template <int U>
__global__ void stream_write_kernel(f32x4 *__restrict__ dst, size_t n) {
  const size_t lanes = (size_t)gridDim.x * blockDim.x;
  const f32x4 z = {1.f, 2.f, 3.f, 4.f};
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += U * lanes) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * lanes < n) __builtin_nontemporal_store(z, &dst[i + u * lanes]);
  }
}

template <int U>
__global__ void stream_copy_kernel(const f32x4 *__restrict__ src, f32x4 *__restrict__ dst,
                                   size_t n) {
  const size_t lanes = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += U * lanes) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * lanes < n) v[u] = __builtin_nontemporal_load(&src[i + u * lanes]);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * lanes < n) __builtin_nontemporal_store(v[u], &dst[i + u * lanes]);
  }
}

// Each workgroup reads the same L2-resident buffer `reps` times, eight
// independent 16-byte loads in flight per lane.  n is a multiple of 8 x blockDim.
__global__ void l2_read_kernel(const float4 *__restrict__ src, size_t n, int reps, float *out) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < reps; ++r)
    for (size_t i = threadIdx.x; i < n; i += 8 * blockDim.x) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[i + u * blockDim.x];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += v[u].x + v[u].y + v[u].z + v[u].w;
    }
  float t = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) t += acc[u];
  if (t == 12345.f) out[blockIdx.x] = t;
}

// LDS read rate: 4 waves each issue `iters` x 8 ds_read_b128 in which lane
// l reads 16 bytes at (l % 16) * rs + (l / 16) * 16 (16 consecutive records
// of stride rs, one 16-byte column per lane group: the A-operand read of the
// kernels).  Offsets vary with the iteration in steps of 8 KiB, which keeps
// the bank mapping; all addresses stay below 64 KiB.
__global__ void lds_read_kernel(int rs, int iters, unsigned long long *cyc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[65536];
  for (int i = threadIdx.x; i < 65536 / 16; i += blockDim.x)
    reinterpret_cast<u32x4 *>(lds)[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
  __syncthreads();
  const int l = threadIdx.x & 63;
  const unsigned addr = (l % 16) * rs + (l / 16) * 16;  // <= 15 * 272 + 48
  __syncthreads();
  const unsigned long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = *reinterpret_cast<const u32x4 *>(lds + addr + (it & 3) * 8192 + u * 2048);
#pragma unroll
    for (int u = 0; u < 8; ++u) asm volatile("" ::"v"(v[u]));
  }
  const unsigned long long t1 = clock64();
  if (threadIdx.x == 0) cyc[0] = t1 - t0;
}

// Vector-ALU issue rate: 16 waves (four per SIMD) each run `iters` x 8
// independent 32-bit integer adds; wave 0 times its loop.  With four waves
// per SIMD the SIMD's issue rate, not a wave's dependency chain, sets the
// time: clocks per wave instruction per SIMD = cyc / (iters * 8 * 4).
__global__ void valu_kernel(int iters, int seed, long long *cyc, int *sink) {
  int a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (int)threadIdx.x * 7 + i + seed;
  __syncthreads();
  const unsigned long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] += seed + i;
    asm volatile("" ::: "memory");
  }
  const unsigned long long t1 = clock64();
  int acc = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc += a[i];
  if (threadIdx.x == 0) cyc[0] = t1 - t0;
  if (acc == 0x7fffffff) sink[0] = acc;
}

// Burst read of one shared buffer by every CU at once: one 256-lane
// workgroup per CU loads `n16` 16-byte pieces of the same buffer (all
// issued before any is used), the pattern of a persistent kernel fetching
// its filter fragments.  Each workgroup records the shader clocks from
// before its first load to after every lane has its data.
__global__ void burst_kernel(const u32x4 *__restrict__ src, int n16, long long *cyc, int *sink) {
  constexpr int kPer = 36;  // loads per lane, issued together
  __syncthreads();
  const long long t0 = clock64();
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int base = 0; base < n16; base += 256 * kPer) {
    u32x4 v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = min(base + i * 256 + (int)threadIdx.x, n16 - 1);
      v[i] = src[idx];
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) acc += v[i];
  }
  asm volatile("" ::"v"(acc));
  __syncthreads();
  const long long t1 = clock64();
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
  if (acc[0] == 0x12345678u && acc[1] == 7u) sink[0] = 1;
}

// Sustained shader clock under a full MFMA load: every CU runs four waves of
// dependent-free f32 MFMAs for `iters` iterations; wave 0 of workgroup 0
// reads the shader clock and the 100 MHz clock around its loop.
__global__ void mfma_clock_kernel(int iters, long long *out, float *sink) {
  f32x4 acc[4] = {};
  const float a = (float)threadIdx.x * 1e-3f, b = 1.0f;
  const long long c0 = clock64(), w0 = wall_clock64();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
  const long long c1 = clock64(), w1 = wall_clock64();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = w1 - w0;
  }
  float t = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) t += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  if (t == -1.0f) sink[0] = t;
}

// Shader clock over the 100 MHz constant clock.
__global__ void clock_kernel(long long *out, int spins) {
  if (threadIdx.x != 0) return;
  const long long c0 = clock64(), w0 = wall_clock64();
  volatile float x = 1.0f;
  for (int i = 0; i < spins; ++i) x = x * 1.0000001f;
  const long long c1 = clock64(), w1 = wall_clock64();
  out[0] = c1 - c0;
  out[1] = w1 - w0;
}

template <class F>
int time_us(F launch, int reps, double *us) {
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int i = 0; i < 3; ++i) launch();
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(a, 0));
  for (int i = 0; i < reps; ++i) launch();
  CK(hipEventRecord(b, 0));
  CK(hipEventSynchronize(b));
  float ms = 0;
  CK(hipEventElapsedTime(&ms, a, b));
  *us = 1000.0 * ms / reps;
  CK(hipGetLastError());
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
  return 0;
}

// A single random cycle through n entries (Sattolo), laid out kStride apart.
std::vector<int> make_cycle(int n, uint64_t seed) {
  std::vector<int> perm(n);
  std::iota(perm.begin(), perm.end(), 0);
  std::mt19937_64 g(seed);
  for (int i = n - 1; i > 0; --i) {
    std::uniform_int_distribution<int> d(0, i - 1);
    std::swap(perm[i], perm[d(g)]);
  }
  std::vector<int> next((size_t)n * kStride, 0);
  for (int i = 0; i < n; ++i) next[(size_t)i * kStride] = perm[i];
  return next;
}

}  // namespace

int main() {
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;

  // shader clock
  long long *dclk;
  CK(hipMalloc(&dclk, 2 * sizeof(long long)));
  hipLaunchKernelGGL(clock_kernel, dim3(1), dim3(64), 0, 0, dclk, 2000000);
  CK(hipDeviceSynchronize());
  long long clk[2];
  CK(hipMemcpy(clk, dclk, sizeof(clk), hipMemcpyDeviceToHost));
  const double ghz = (double)clk[0] / (double)clk[1] * 0.1;

  // launch cost in a back-to-back stream
  double t_launch;
  if (time_us([&] { hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0, nullptr); }, 2000,
              &t_launch))
    return 1;
  double t_launch_full;  // a grid that covers every CU
  if (time_us([&] { hipLaunchKernelGGL(empty_kernel, dim3(4 * cus), dim3(256), 0, 0, nullptr); },
              2000, &t_launch_full))
    return 1;

  // per-kernel cost inside a captured graph: 200 launches of an empty
  // single-workgroup kernel, and of a full-grid one, replayed
  double t_graph = 0, t_graph_full = 0;
  for (int full = 0; full < 2; ++full) {
    hipStream_t st;
    CK(hipStreamCreate(&st));
    hipGraph_t graph;
    hipGraphExec_t exec;
    CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int i = 0; i < 200; ++i)
      hipLaunchKernelGGL(empty_kernel, dim3(full ? 4 * cus : 1), dim3(full ? 256 : 64), 0, st, nullptr);
    CK(hipStreamEndCapture(st, &graph));
    CK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    CK(hipGraphLaunch(exec, st));
    CK(hipStreamSynchronize(st));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a, st));
    for (int r = 0; r < 10; ++r) CK(hipGraphLaunch(exec, st));
    CK(hipEventRecord(b, st));
    CK(hipEventSynchronize(b));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, a, b));
    (full ? t_graph_full : t_graph) = 1000.0 * ms / (10 * 200);
    CK(hipGraphExecDestroy(exec));
    CK(hipGraphDestroy(graph));
    CK(hipStreamDestroy(st));
  }

  // dependent-load latency: HBM (1 GiB span), L2 (1 MiB span)
  int *dout;
  CK(hipMalloc(&dout, 4 * cus * 64 * sizeof(int)));
  const int n_hbm = (1 << 30) / (kStride * 4), n_l2 = (1 << 20) / (kStride * 4);
  const int hops = 4000;
  double lat_hbm, lat_l2, lat_loaded, lat_l2_loaded;
  {
    std::vector<int> next = make_cycle(n_hbm, 1);
    int *d;
    CK(hipMalloc(&d, next.size() * sizeof(int)));
    CK(hipMemcpy(d, next.data(), next.size() * sizeof(int), hipMemcpyHostToDevice));
    double us;
    if (time_us([&] { hipLaunchKernelGGL(chase_kernel, dim3(1), dim3(64), 0, 0, d, hops, n_hbm, dout); },
                3, &us))
      return 1;
    lat_hbm = us / hops;
    // every CU chasing at once, 4 waves each
    if (time_us([&] { hipLaunchKernelGGL(chase_kernel, dim3(4 * cus), dim3(64), 0, 0, d, hops, n_hbm, dout); },
                3, &us))
      return 1;
    lat_loaded = us / hops;
    CK(hipFree(d));
  }
  {
    std::vector<int> next = make_cycle(n_l2, 2);
    int *d;
    CK(hipMalloc(&d, next.size() * sizeof(int)));
    CK(hipMemcpy(d, next.data(), next.size() * sizeof(int), hipMemcpyHostToDevice));
    double us;
    if (time_us([&] { hipLaunchKernelGGL(chase_kernel, dim3(1), dim3(64), 0, 0, d, hops, n_l2, dout); },
                3, &us))
      return 1;
    lat_l2 = us / hops;
    // every CU chasing at once through the same L2-resident span
    if (time_us([&] { hipLaunchKernelGGL(chase_kernel, dim3(4 * cus), dim3(64), 0, 0, d, hops, n_l2, dout); },
                3, &us))
      return 1;
    lat_l2_loaded = us / hops;
    CK(hipFree(d));
  }

  // LDS: clocks per ds_read_b128 wave instruction, four waves reading, for
  // record strides of 16 mod 64 bytes (80, 144), 32 mod 64 (96, 160) and 128
  const int strides[5] = {80, 96, 128, 144, 160};
  double lds_clk[5];
  unsigned long long *dcyc;
  CK(hipMalloc(&dcyc, sizeof(unsigned long long)));
  for (int i = 0; i < 5; ++i) {
    const int iters = 200;
    hipLaunchKernelGGL(lds_read_kernel, dim3(1), dim3(256), 0, 0, strides[i], iters, dcyc);
    CK(hipDeviceSynchronize());
    unsigned long long c = 0;
    CK(hipMemcpy(&c, dcyc, sizeof c, hipMemcpyDeviceToHost));
    lds_clk[i] = (double)c / (iters * 8);
  }
  CK(hipFree(dcyc));

  // HBM copy bandwidth, 1 GiB each way
  const size_t bytes = (size_t)1 << 30;
  float4 *src, *dst;
  CK(hipMalloc(&src, bytes));
  CK(hipMalloc(&dst, bytes));
  CK(hipMemset(src, 0, bytes));
  double t_copy;
  if (time_us([&] { hipLaunchKernelGGL(copy_kernel, dim3(8 * cus), dim3(256), 0, 0, src, dst, bytes / 16); },
              10, &t_copy))
    return 1;
  const double copy_gbs = 2.0 * bytes / (t_copy * 1e3);

  // Attainable HBM rate: the streaming kernels over 1 GiB, best over grids
  // of 4..32 workgroups per CU and 4 or 8 accesses in flight per lane.
  double best_read = 0, best_write = 0, best_copy = 0;
  int best_read_cfg = 0, best_write_cfg = 0, best_copy_cfg = 0;
  float *rsink;
  CK(hipMalloc(&rsink, 64 * cus * sizeof(float)));
  const size_t n16 = bytes / 16;
  for (int per_cu : {4, 8, 16, 32})
    for (int u : {4, 8}) {
      const dim3 g(per_cu * cus), b(256);
      double t;
      if (time_us([&] {
            if (u == 4) hipLaunchKernelGGL(stream_read_kernel<4>, g, b, 0, 0, reinterpret_cast<const f32x4 *>(src), n16, rsink);
            else hipLaunchKernelGGL(stream_read_kernel<8>, g, b, 0, 0, reinterpret_cast<const f32x4 *>(src), n16, rsink);
          }, 10, &t))
        return 1;
      if (bytes / (t * 1e3) > best_read) best_read = bytes / (t * 1e3), best_read_cfg = per_cu * 10 + u;
      if (time_us([&] {
            if (u == 4) hipLaunchKernelGGL(stream_write_kernel<4>, g, b, 0, 0, reinterpret_cast<f32x4 *>(dst), n16);
            else hipLaunchKernelGGL(stream_write_kernel<8>, g, b, 0, 0, reinterpret_cast<f32x4 *>(dst), n16);
          }, 10, &t))
        return 1;
      if (bytes / (t * 1e3) > best_write) best_write = bytes / (t * 1e3), best_write_cfg = per_cu * 10 + u;
      if (time_us([&] {
            if (u == 4) hipLaunchKernelGGL(stream_copy_kernel<4>, g, b, 0, 0, reinterpret_cast<const f32x4 *>(src), reinterpret_cast<f32x4 *>(dst), n16);
            else hipLaunchKernelGGL(stream_copy_kernel<8>, g, b, 0, 0, reinterpret_cast<const f32x4 *>(src), reinterpret_cast<f32x4 *>(dst), n16);
          }, 10, &t))
        return 1;
      if (2.0 * bytes / (t * 1e3) > best_copy) best_copy = 2.0 * bytes / (t * 1e3), best_copy_cfg = per_cu * 10 + u;
    }
  CK(hipFree(rsink));

  // per-CU read rate from L2: one 1024-lane workgroup per CU, 256 KiB buffer
  // read 64 times (l2n is a multiple of 8 x 1024)
  const size_t l2n = (256 << 10) / 16;
  const int reps = 64;
  float *dsink;
  CK(hipMalloc(&dsink, cus * 4 * sizeof(float)));
  double t_l2;
  if (time_us([&] { hipLaunchKernelGGL(l2_read_kernel, dim3(cus), dim3(1024), 0, 0, src, l2n, reps, dsink); },
              5, &t_l2))
    return 1;
  const double l2_bytes_per_clk_cu = (double)l2n * 16 * reps / (t_l2 * 1e3 * ghz);

  // vector-ALU issue rate: one CU with four waves per SIMD (the SIMD's
  // rate), and with one wave per SIMD (a single wave's rate)
  double valu_clk = 0, wave_valu_clk = 0;
  {
    const int iters = 4096;
    int *dint;
    CK(hipMalloc(&dint, sizeof(int)));
    for (int waves_per_simd : {4, 1}) {
      for (int rep = 0; rep < 2; ++rep)
        hipLaunchKernelGGL(valu_kernel, dim3(1), dim3(256 * waves_per_simd), 0, 0, iters, 3, dclk, dint);
      CK(hipDeviceSynchronize());
      long long c = 0;
      CK(hipMemcpy(&c, dclk, sizeof c, hipMemcpyDeviceToHost));
      (waves_per_simd == 4 ? valu_clk : wave_valu_clk) = (double)c / (iters * 8.0 * waves_per_simd);
    }
    CK(hipFree(dint));
  }

  // burst read of a shared 147456-byte buffer by every CU (the filter
  // fragments of a 64-filter f32 3x3 workgroup): median over the CUs
  double burst_bytes_per_clk_cu = 0;
  {
    const int n16 = 147456 / 16;
    int *dint;
    long long *dcyc;
    CK(hipMalloc(&dint, sizeof(int)));
    CK(hipMalloc(&dcyc, cus * sizeof(long long)));
    for (int rep = 0; rep < 3; ++rep)
      hipLaunchKernelGGL(burst_kernel, dim3(cus), dim3(256), 0, 0,
                         reinterpret_cast<const u32x4 *>(src), n16, dcyc, dint);
    CK(hipDeviceSynchronize());
    std::vector<long long> cyc(cus);
    CK(hipMemcpy(cyc.data(), dcyc, cus * sizeof(long long), hipMemcpyDeviceToHost));
    std::sort(cyc.begin(), cyc.end());
    burst_bytes_per_clk_cu = 147456.0 / (double)cyc[cus / 2];
    CK(hipFree(dint));
    CK(hipFree(dcyc));
  }

  // shader clock sustained under an all-CU MFMA load
  double loaded_ghz = 0;
  {
    float *dsf;
    CK(hipMalloc(&dsf, sizeof(float)));
    for (int rep = 0; rep < 2; ++rep)
      hipLaunchKernelGGL(mfma_clock_kernel, dim3(cus), dim3(256), 0, 0, 200000, dclk, dsf);
    CK(hipDeviceSynchronize());
    long long cw[2];
    CK(hipMemcpy(cw, dclk, sizeof cw, hipMemcpyDeviceToHost));
    loaded_ghz = (double)cw[0] / (double)cw[1] * 0.1;
    CK(hipFree(dsf));
  }

  printf("{\"device\": \"%s\", \"cus\": %d, \"shader_clock_ghz\": %.3f, \"launch_us\": %.3f, "
         "\"launch_full_grid_us\": %.3f, \"graph_launch_us\": %.3f, \"graph_launch_full_grid_us\": %.3f, \"hbm_latency_us\": %.3f, \"hbm_latency_loaded_us\": %.3f, "
         "\"l2_latency_us\": %.3f, \"l2_latency_loaded_us\": %.3f, \"hbm_copy_gbs\": %.1f, \"l2_read_bytes_per_clk_cu\": %.2f, "
         "\"lds_b128_clk_per_wave_instr\": {\"80\": %.1f, \"96\": %.1f, \"128\": %.1f, \"144\": %.1f, \"160\": %.1f}, "
         "\"lds_bytes_per_clk_cu\": %.1f, \"valu_clk_per_wave_instr\": %.2f, \"valu_instr_per_clk_cu\": %.2f, "
         "\"wave_valu_clk\": %.2f, \"burst_bytes_per_clk_cu\": %.1f, \"mfma_loaded_clock_ghz\": %.3f, "
         "\"hbm_stream_read_gbs\": %.1f, \"hbm_stream_write_gbs\": %.1f, \"hbm_stream_copy_gbs\": %.1f, "
         "\"hbm_stream_best_cfg\": {\"read\": \"%d wg/cu x %d\", \"write\": \"%d wg/cu x %d\", \"copy\": \"%d wg/cu x %d\"}}\n",
         prop.gcnArchName, cus, ghz, t_launch, t_launch_full, t_graph, t_graph_full, lat_hbm, lat_loaded, lat_l2, lat_l2_loaded, copy_gbs,
         l2_bytes_per_clk_cu, lds_clk[0], lds_clk[1], lds_clk[2], lds_clk[3], lds_clk[4],
         4.0 * 1024 / lds_clk[4], valu_clk, 4.0 / valu_clk, wave_valu_clk, burst_bytes_per_clk_cu,
         loaded_ghz, best_read, best_write, best_copy, best_read_cfg / 10, best_read_cfg % 10,
         best_write_cfg / 10, best_write_cfg % 10, best_copy_cfg / 10, best_copy_cfg % 10);
  CK(hipFree(src));
  CK(hipFree(dst));
  CK(hipFree(dsink));
  CK(hipFree(dout));
  CK(hipFree(dclk));
  return 0;
}
