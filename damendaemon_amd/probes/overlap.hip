// Hardware probes behind the design notes of the attention kernels (gfx950).
// Not part of the library: `python bench.py --probe` compiles and runs this
// file.  Each probe prints one JSON line.  Rates are per SIMD (1,024 on an
// MI355X), converted to cycles at the shader clock the clock probe measures
// first (MFMA chains on every SIMD), so they are approximate where another
// probe runs at another clock.
//
//   valu_rate     wave-instructions per SIMD and cycle of v_exp_f32 and v_fma_f32
//   mfma_rate     v_mfma_f32_32x32x16_bf16 per SIMD and cycle
//   lds_read      CU read bandwidth of ds_read_b128 and ds_read_b64_tr_b16 with
//                 the lane-contiguous layouts of the prefill kernel (8 waves)
//   tile_step     one prefill tile-step of 8 waves (2 per SIMD): 16 S^T MFMAs +
//                 16 P.V MFMAs (32x32x16) with K / V^T operands from LDS, then the
//                 softmax of 32 scores per lane (fma, exp2, fp16 pack, dot2 row
//                 sums, max), one barrier per step -- the best case of the prefill
//                 kernel's compute, without memory traffic.
//   coissue       how much vector work hides under the matrix cores: waves 0-3
//                 of a CU issue only v_mfma_f32_32x32x16 (4 independent chains),
//                 waves 4-7 only v_fma_f32 or v_exp_f32, k per MFMA; cycles per
//                 MFMA against 32 for the MFMA waves alone
//   tile_step_64  the same tile-step as tile_step with one wave per SIMD owning
//                 64 columns (two column blocks share every K and V^T operand,
//                 half the LDS reads per flop), softmax of the next tile
//                 interleaved with the P.V MFMAs by the compiler
//   clock         shader clock (s_memtime against the 100 MHz s_memrealtime)
//                 while MFMA chains run on every SIMD
#include <hip/hip_runtime.h>
#include <cstdio>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char;

static double kClock = 2.1e9;   // replaced by the measured clock in main()
constexpr int kSimds = 1024;

__device__ __forceinline__ unsigned lds_addr(const void *p) { return (unsigned)(uintptr_t)(const lds_char *)p; }
__device__ __forceinline__ u32x4 rd128(unsigned a, int off) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(off) : "memory");
  return r;
}
__device__ __forceinline__ u32x2 rdtr(unsigned a, int off) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(off) : "memory");
  return r;
}
template <typename T>
__device__ __forceinline__ void lw(T &x, int n) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(n < 15 ? n : 15));
}
template <typename T>
__device__ __forceinline__ void lw2(T &x, T &y, int n) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "i"(n < 15 ? n : 15));
}
__device__ __forceinline__ f32x16 mfs(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
__device__ __forceinline__ f32x16 mfo(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}
__device__ __forceinline__ unsigned cvt(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, f16x2));
}

constexpr int N = 2048;
__global__ void k_exp(float *out, float x0) {
  float a[8];
  for (int i = 0; i < 8; ++i) a[i] = x0 + threadIdx.x * 1e-6f + i;
  for (int it = 0; it < N; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = __builtin_amdgcn_exp2f(a[i]);
  float s = 0;
  for (int i = 0; i < 8; ++i) s += a[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
__global__ void k_fma(float *out, float x0) {
  float a[8];
  for (int i = 0; i < 8; ++i) a[i] = x0 + threadIdx.x * 1e-6f + i;
  for (int it = 0; it < N; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = __builtin_fmaf(a[i], 0.999f, 0.001f);
  float s = 0;
  for (int i = 0; i < 8; ++i) s += a[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
__global__ void k_mfma(float *out, float x0) {
  f32x16 acc[4] = {};
  u32x4 a = {threadIdx.x, 1u, 2u, 3u}, b = {5u, 6u, 7u, (unsigned)x0};
  for (int it = 0; it < N / 4; ++it)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = mfs(a, b, acc[i]);
  float s = 0;
  for (int i = 0; i < 4; ++i) s += acc[i][0] + acc[i][7];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
template <int MODE>  // 1: ds_read_b128, 2: ds_read_b64_tr_b16
__global__ __launch_bounds__(512) void k_lds(unsigned *out) {
  __shared__ __attribute__((aligned(1024))) char sm[65536];
  for (int i = threadIdx.x; i < 16384; i += 512) ((unsigned *)sm)[i] = i;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const unsigned ka = lds_addr(sm) + 1024u * 4 * ((lane >> 4) & 1) + 16u * (lane & 15) + 256u * (lane >> 5);
  const unsigned va = lds_addr(sm) + 32768 + 8u * lane;
  unsigned acc = 0;
  for (int t = 0; t < 512; ++t) {
    if (MODE == 1) {
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        u32x4 a = rd128(ka, (i / 2) * 1024), b = rd128(ka, (i / 2) * 1024 + 512), c = rd128(ka, (i / 2 + 1) * 1024),
              d = rd128(ka, (i / 2 + 1) * 1024 + 512);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        acc ^= a[0] ^ b[1] ^ c[2] ^ d[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; i += 8) {
        u32x2 r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = rdtr(va, ((i + j) * 512) % 16384);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= r[j][0] + r[j][1];
      }
    }
  }
  out[blockIdx.x * 512 + threadIdx.x] = acc;
}
constexpr int kTiles = 128;
__global__ __launch_bounds__(512) void k_tile(float *out, float x0) {
  __shared__ __attribute__((aligned(1024))) char sm[65536];
  for (int i = threadIdx.x; i < 16384; i += 512) ((unsigned *)sm)[i] = 0x3c003c00u + (i & 7);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const unsigned kb = lds_addr(sm) + 1024u * 4 * ((lane >> 4) & 1) + 16u * (lane & 15) + 256u * (lane >> 5);
  const unsigned vb = lds_addr(sm) + 32768 + 8u * lane;
  u32x4 q[8];
  for (int i = 0; i < 8; ++i) q[i] = u32x4{threadIdx.x * 3u + i, 1u, 2u, 4u};
  f32x16 o[4] = {}, s[2] = {};
  u32x4 pp[2][2];
  for (int b = 0; b < 2; ++b)
    for (int j = 0; j < 2; ++j) pp[b][j] = u32x4{1u, 2u, 3u, threadIdx.x};
  float l = 0.f, mu = x0;
  for (int t = 0; t < kTiles; ++t) {
    constexpr int NS = 16, NM = 32, R = 4;
    u32x4 kop[R];
    u32x2 lo[R], hi[R];
    auto rd = [&](int i) {
      if (i < NS) {
        kop[i % R] = rd128(kb, (2 * (i & 1) * 4 + (i >> 1) / 2) * 1024 + 512 * ((i >> 1) & 1));
      } else {
        lo[i % R] = rdtr(vb, 2 * (i - NS) * 512);
        hi[i % R] = rdtr(vb, 2 * (i - NS) * 512 + 512);
      }
    };
    auto after = [](int i) constexpr {
      int n = 0;
      for (int j = i + 1; j < i + R && j < NM; ++j) n += j < NS ? 1 : 2;
      return n;
    };
#pragma unroll
    for (int i = 0; i < R; ++i) rd(i);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i < NS) {
        lw(kop[i % R], after(i));
        s[i & 1] = mfs(kop[i % R], q[i >> 1], i < 2 ? f32x16{} : s[i & 1]);
      } else {
        const int j = i - NS;
        lw2(lo[i % R], hi[i % R], after(i));
        o[j & 3] = mfo(u32x4{lo[i % R][0], lo[i % R][1], hi[i % R][0], hi[i % R][1]}, pp[j >> 3][(j >> 2) & 1],
                       o[j & 3]);
      }
      if (i + R < NM) rd(i + R);
    }
    float mx = s[0][0];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; r += 2) mx = fmaxf(fmaxf(mx, s[b][r]), s[b][r + 1]);
    mu = fmaxf(mx, mu) * 0.1f;
    float lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = i >> 3, r = 2 * (i & 7);
      const unsigned h = cvt(__builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r], 0.1f, -mu)),
                             __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r + 1], 0.1f, -mu)));
      pp[b][(i & 7) >> 2][i & 3] = h;
      lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, h), f16x2{(_Float16)1.f, (_Float16)1.f}, lsum, false);
    }
    l += lsum;
    asm volatile("s_barrier" ::: "memory");
  }
  float r = l;
  for (int m = 0; m < 4; ++m) r += o[m][0] + o[m][5];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// waves 0-3: MFMA chains; waves 4-7: NV vector ops (fma, or exp when EXP) per MFMA
template <int NV, int EXP>
__global__ __launch_bounds__(512) void k_coissue(float *out, int n, float x0) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float s = 0;
  if (w < 4) {
    f32x16 acc[4] = {};
    const u32x4 a = {threadIdx.x, 1u, 2u, 3u}, b = {5u, 6u, 7u, (unsigned)x0};
    for (int it = 0; it < n; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = mfs(a, b, acc[j]);
    for (int j = 0; j < 4; ++j) s += acc[j][0] + acc[j][5];
  } else if (NV > 0) {
    float v[8];
    for (int i = 0; i < 8; ++i) v[i] = x0 + i + threadIdx.x;
    for (int it = 0; it < n; ++it)
#pragma unroll
      for (int u = 0; u < 4 * NV; ++u)
        v[u % 8] = EXP ? __builtin_amdgcn_exp2f(v[u % 8]) : __builtin_fmaf(v[u % 8], 0.999f, 0.5f);
    for (int i = 0; i < 8; ++i) s += v[i];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// one wave per SIMD, 64 columns per wave
__global__ __launch_bounds__(256) void k_tile64(float *out, float x0) {
  __shared__ __attribute__((aligned(1024))) char sm[65536];
  for (int i = threadIdx.x; i < 16384; i += 256) ((unsigned *)sm)[i] = 0x3c003c00u + (i & 7);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const unsigned kb = lds_addr(sm) + 1024u * 4 * ((lane >> 4) & 1) + 16u * (lane & 15) + 256u * (lane >> 5);
  const unsigned vb = lds_addr(sm) + 32768 + 8u * lane;
  u32x4 q[2][8];
  for (int c = 0; c < 2; ++c)
    for (int i = 0; i < 8; ++i) q[c][i] = u32x4{threadIdx.x * 3u + i + c, 1u, 2u, 4u};
  f32x16 o[2][4] = {}, s[2][2] = {};
  u32x4 pp[2][2][2];
  for (int c = 0; c < 2; ++c)
    for (int b = 0; b < 2; ++b)
      for (int j = 0; j < 2; ++j) pp[c][b][j] = u32x4{1u, 2u, 3u, threadIdx.x};
  float l[2] = {0.f, 0.f}, mu[2] = {x0, x0};
  for (int t = 0; t < kTiles; ++t) {
    {
      constexpr int R = 4;
      u32x4 kop[R];
      auto rd = [&](int i) { kop[i % R] = rd128(kb, (2 * (i & 1) * 4 + (i >> 1) / 2) * 1024 + 512 * ((i >> 1) & 1)); };
#pragma unroll
      for (int i = 0; i < R; ++i) rd(i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        lw(kop[i % R], i + R - 1 < 16 ? R - 1 : 15 - i);
        const int cc = i >> 1, b = i & 1;
        s[0][b] = mfs(kop[i % R], q[0][cc], cc == 0 ? f32x16{} : s[0][b]);
        s[1][b] = mfs(kop[i % R], q[1][cc], cc == 0 ? f32x16{} : s[1][b]);
        if (i + R < 16) rd(i + R);
      }
    }
    float mx[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float m = s[c][0][0];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; r += 2) m = fmaxf(fmaxf(m, s[c][b][r]), s[c][b][r + 1]);
      mx[c] = m;
    }
    {
      constexpr int R = 4;
      u32x2 lo[R], hi[R];
      auto rd = [&](int j) {
        lo[j % R] = rdtr(vb, 2 * j * 512);
        hi[j % R] = rdtr(vb, 2 * j * 512 + 512);
      };
#pragma unroll
      for (int j = 0; j < R; ++j) rd(j);
      u32x4 np[2][2][2];
      float ls[2] = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        lw2(lo[j % R], hi[j % R], j + R - 1 < 16 ? 2 * (R - 1) : 2 * (15 - j));
        const u32x4 op = {lo[j % R][0], lo[j % R][1], hi[j % R][0], hi[j % R][1]};
        const int md = j & 3, bj = j >> 2;
        o[0][md] = mfo(op, pp[0][bj >> 1][bj & 1], o[0][md]);
        o[1][md] = mfo(op, pp[1][bj >> 1][bj & 1], o[1][md]);
        if (j + R < 16) rd(j + R);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int pi = 2 * j + h, c = pi >> 4, i = pi & 15, b = i >> 3, r = 2 * (i & 7);
          const float m0 = fmaxf(mx[c], mu[c]) * 0.1f;
          const unsigned hh = cvt(__builtin_amdgcn_exp2f(__builtin_fmaf(s[c][b][r], 0.1f, -m0)),
                                  __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][b][r + 1], 0.1f, -m0)));
          np[c][b][(i & 7) >> 2][i & 3] = hh;
          ls[c] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, hh), f16x2{(_Float16)1.f, (_Float16)1.f}, ls[c],
                                         false);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        l[c] += ls[c];
        mu[c] = fmaxf(mx[c], mu[c]);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) pp[c][b][jj] = np[c][b][jj];
      }
    }
    asm volatile("s_barrier" ::: "memory");
  }
  float r = l[0] + l[1];
  for (int c = 0; c < 2; ++c)
    for (int m = 0; m < 4; ++m) r += o[c][m][0] + o[c][m][5];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

__global__ __launch_bounds__(512) void k_clock(unsigned long long *ticks, int n) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc[4] = {};
  const u32x4 a = {threadIdx.x, 1u, 2u, 3u}, b = {5u, 6u, 7u, 8u};
  for (int it = 0; it < n; ++it)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfs(a, b, acc[j]);
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0;
  for (int j = 0; j < 4; ++j) s += acc[j][0] + acc[j][5];
  if (threadIdx.x == 0) {
    ticks[2 * blockIdx.x] = c1 - c0;
    ticks[2 * blockIdx.x + 1] = (r1 - r0) | (s == 1.2345f ? 1ull << 63 : 0ull);
  }
}

template <typename F>
float time_ms(F launch) {
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  launch();
  (void)hipDeviceSynchronize();
  (void)hipEventRecord(e0);
  for (int r = 0; r < 5; ++r) launch();
  (void)hipEventRecord(e1);
  (void)hipEventSynchronize(e1);
  float ms;
  (void)hipEventElapsedTime(&ms, e0, e1);
  return ms / 5;
}

int main() {
  float *o;
  if (hipMalloc(&o, 256 * 1024 * 4) != hipSuccess) return 1;
  unsigned long long *ticks;
  if (hipMalloc(&ticks, 256 * 16) != hipSuccess) return 1;
  unsigned long long h[2];
  k_clock<<<256, 512>>>(ticks, 20000);   // warm
  if (hipDeviceSynchronize() != hipSuccess) return 1;
  k_clock<<<256, 512>>>(ticks, 20000);
  if (hipMemcpy(h, ticks, 16, hipMemcpyDeviceToHost) != hipSuccess) return 1;
  kClock = h[0] / (double)((h[1] & ~(1ull << 63)) * 10) * 1e9;
  printf("{\"probe\": \"clock\", \"shader_mhz_under_mfma\": %.0f}\n", kClock * 1e-6);
  const int blocks = 256, thr = 512;  // two waves per SIMD
  const double waves_per_simd = blocks * thr / 64.0 / kSimds;
  const float te = time_ms([&] { k_exp<<<blocks, thr>>>(o, 1.f); });
  const float tf = time_ms([&] { k_fma<<<blocks, thr>>>(o, 1.f); });
  const float tm = time_ms([&] { k_mfma<<<blocks, thr>>>(o, 1.f); });
  auto cyc_per = [&](float ms, double instrs_per_wave) { return ms * 1e-3 * kClock / (waves_per_simd * instrs_per_wave); };
  printf("{\"probe\": \"valu_rate\", \"cycles_per_v_exp_f32\": %.2f, \"cycles_per_v_fma_f32\": %.2f}\n",
         cyc_per(te, N * 8.0), cyc_per(tf, N * 8.0));
  printf("{\"probe\": \"mfma_rate\", \"cycles_per_mfma_32x32x16_bf16\": %.2f}\n", cyc_per(tm, N));
  const float tl1 = time_ms([&] { k_lds<1><<<256, 512>>>((unsigned *)o); });
  const float tl2 = time_ms([&] { k_lds<2><<<256, 512>>>((unsigned *)o); });
  auto bw = [&](float ms) { return 8 * 16384.0 * 512 / (ms * 1e-3 * kClock / 1.0); };  // bytes per CU-cycle
  printf("{\"probe\": \"lds_read\", \"bytes_per_cu_cycle_b128\": %.0f, \"bytes_per_cu_cycle_tr_b16\": %.0f}\n", bw(tl1),
         bw(tl2));
  const float tt = time_ms([&] { k_tile<<<256, 512>>>(o, 1.f); });
  const double step = tt * 1e-3 * kClock / kTiles;
  printf("{\"probe\": \"tile_step\", \"cycles_per_8_wave_tile_step\": %.0f, \"mfma_cycles\": 2048, \"mfma_busy\": %.3f}\n",
         step, 2048.0 / step);
  auto coissue = [&](auto launch, const char *what, int k) {
    const int n = 2000;
    const float ms = time_ms([&] { launch(n); });
    printf("{\"probe\": \"coissue\", \"vector_op\": \"%s\", \"per_mfma\": %d, \"cycles_per_mfma\": %.1f}\n", what, k,
           ms * 1e-3 * kClock / (n * 4.0));
  };
  coissue([&](int n) { k_coissue<0, 0><<<256, 512>>>(o, n, 1.f); }, "none", 0);
  coissue([&](int n) { k_coissue<4, 0><<<256, 512>>>(o, n, 1.f); }, "v_fma_f32", 4);
  coissue([&](int n) { k_coissue<8, 0><<<256, 512>>>(o, n, 1.f); }, "v_fma_f32", 8);
  coissue([&](int n) { k_coissue<2, 1><<<256, 512>>>(o, n, 1.f); }, "v_exp_f32", 2);
  coissue([&](int n) { k_coissue<4, 1><<<256, 512>>>(o, n, 1.f); }, "v_exp_f32", 4);
  const float t64 = time_ms([&] { k_tile64<<<256, 256>>>(o, 1.f); });
  const double step64 = t64 * 1e-3 * kClock / kTiles;
  printf("{\"probe\": \"tile_step_64\", \"cycles_per_4_wave_tile_step\": %.0f, \"mfma_cycles\": 2048, \"mfma_busy\": %.3f}\n",
         step64, 2048.0 / step64);
  return 0;
}
