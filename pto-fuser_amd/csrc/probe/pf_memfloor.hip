// Memory floor of the scan kernels' access patterns on gfx950: a measurement probe, not part of
// libptofuser_hip (built as its own executable next to the library).
//
// Each stage-2 scan workgroup (one chain x one column slice, one workgroup per CU) streams a
// chunk image per step from HBM through registers into a double-buffered LDS stage (its loader
// waves: three rotating register sets, a chunk's loads issued three steps ahead, one LDS store
// per 16-byte vector) and writes its o rows.  The column slices of one chain sit on one XCD and
// read the same image.  This probe runs exactly that traffic with no compute: 256 workgroups of
// four loader waves, SH workgroups on an XCD (blockIdx % 8) sharing each image, OB bytes of o rows
// per workgroup and step (each slice OB / 64 bytes of every token's row, non-temporal or
// through the cache as the kernel stores them).  The time per step is the shortest chunk period
// those loads and stores allow; it is printed for each kernel's pattern with the loads alone and
// the stores alone beside it, together with the shader clock the probe ran at (s_memtime against
// s_memrealtime's 100 MHz).
//
// A second form replays the kernels' own address pattern: the chunk images read from tensors laid
// out as the kernels read them (k, q, v and o as [B*H, T, 128], T as [B*H, NC, 64, 64]; KDA's
// W, QE, KB as [B*H, NC, 64, 128], T diag(beta) as [B*H, NC, 64, 64], v as [B*H, T, 128],
// the decay as [B*H, NC, 128] fp32), with the kernels' chain-to-workgroup mapping (the slices of
// a chain on one XCD) and each loader lane's 16-byte vectors, so the floor includes what the
// tensors' strides (powers of two at these shapes) cost the memory system.
//
// Every offset stays inside its buffer (descriptors carry each region's size; steps clamp).
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSteps = 96;        // chunks streamed per launch
constexpr int kGroups = 256;      // one workgroup per CU
constexpr int kMaxKiB = 64;       // largest chunk image (LDS: two stages)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// KIB: 16-byte loads per workgroup and chunk (KiB, a multiple of 4: wave w loads the 1 KiB
// vectors w, w + 4, ..., every wave the same number, with no branch around a load, as the
// kernels' loaders do; where a kernel's lanes repeat a vector, the repeat is counted);
// SH: workgroups sharing one image; OB: o bytes per workgroup and step (0: none); NTST: o stores
// non-temporal; LD: issue the loads.
template <int KIB, int SH, int OB, bool NTST, bool LD>
__global__ __launch_bounds__(256) void floor_kernel(const unsigned char* src, unsigned char* dst,
                                                    uint32_t* sink, unsigned long long* clocks) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][kMaxKiB * 1024];
  static_assert(KIB % 4 == 0 && KIB <= kMaxKiB, "chunk image: whole 4 KiB rounds");
  constexpr int N = KIB / 4;                          // 1 KiB loads per wave and step
  constexpr uint32_t kStep = KIB * 1024;
  constexpr uint32_t kRegion = kStep * kSteps;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int x = blockIdx.x % 8, i = blockIdx.x / 8;
  const int region = x * (32 / SH) + i / SH;          // the chain this workgroup's slice reads
  const int slice = i % SH;
  const __amdgpu_buffer_rsrc_t r = rsrc(src + (size_t)region * kRegion, kRegion);
  constexpr uint32_t kOBytes = (OB > 0 ? OB : 64) * SH * kSteps;   // o rows of one chain
  const __amdgpu_buffer_rsrc_t ro = rsrc(dst + (size_t)region * kOBytes, kOBytes);

  struct Set { u32x4 v[N]; };
  auto load = [&](Set& s, int step) {
    if constexpr (LD) {
#pragma unroll
      for (int k = 0; k < N; ++k)
        s.v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, 16 * lane, (uint32_t)step * kStep + (4 * k + w) * 1024, 0);
    }
  };
  auto stage = [&](int buf, const Set& s) {
#pragma unroll
    for (int k = 0; k < N; ++k) *reinterpret_cast<u32x4*>(lds[buf] + (4 * k + w) * 1024 + 16 * lane) = s.v[k];
  };
  auto ostore = [&](int step) {
    if constexpr (OB > 0) {
      // 64 tokens per step; this slice's BPT bytes of each token's (BPT * SH)-byte row; a store
      // instruction covers 1 KiB (TPI tokens), wave w tokens 16 w .. 16 w + 15
      constexpr int BPT = OB / 64, LPT = BPT / 16, TPI = 64 / LPT;
      const u32x4 val = {(uint32_t)step, 1u, 2u, 3u};
#pragma unroll
      for (int k = 0; k < 16 / TPI; ++k) {
        const uint32_t tok = (uint32_t)step * 64 + 16 * w + TPI * k + lane / LPT;
        __builtin_amdgcn_raw_buffer_store_b128(val, ro, tok * BPT * SH + BPT * slice + 16 * (lane % LPT), 0,
                                               NTST ? 2 : 0);
      }
    }
  };
  uint32_t acc = 0;
  auto interval = [&](Set& ld, const Set& nx, int j) {
    load(ld, min(j + 3, kSteps - 1));
    stage((j + 1) & 1, nx);
    ostore(j);
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);               // LDS stores landed; loads stay in flight
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
    acc += lds[j & 1][(threadIdx.x * 16) % kStep];
  };
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  Set s0, s1, s2;
  load(s0, 0);
  load(s1, 1);
  load(s2, 2);
  stage(0, s0);
  __syncthreads();
  interval(s0, s1, 0);
  for (int j = 1; j + 3 < kSteps; j += 3) {
    interval(s1, s2, j);
    interval(s2, s0, j + 1);
    interval(s0, s1, j + 2);
  }
  sink[blockIdx.x * 256 + threadIdx.x] = acc;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clocks[0] = __builtin_amdgcn_s_memtime() - t0;
    clocks[1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

constexpr int executed_steps(int steps = kSteps) {
  int n = 1;
  for (int j = 1; j + 3 < steps; j += 3) n += 3;
  return n;
}

// Tensors of one workload in the kernels' layout.
struct Tensors {
  const unsigned char* a[6];   // GDN: k, q, T, v; KDA: W, QE, KB, v, decay, T diag(beta)
  unsigned char* o;            // [chains, T, 128] fp32
};

// The kernels' traffic at their own addresses.  KDA false: GDN stage 2 (per loader wave and
// chunk 4 k, 4 q, 2 T vectors of 1 KiB and one v load per lane); KDA true: 4 W, 4 QE, 4 KB,
// 2 T diag(beta), one v and one decay load per lane.  NCOL: columns per slice (32 or 16), NC: chunks per chain,
// STEPS: chunks streamed, NTST: o stores non-temporal, LD / ST: issue the loads / the stores.
template <bool KDA, int NCOL, int NC, int STEPS, bool NTST, bool LD, bool ST>
__global__ __launch_bounds__(256) void layout_kernel(Tensors t, uint32_t* sink, int chains) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][kMaxKiB * 1024];
  constexpr int NS = 128 / NCOL;                    // slices per chain
  constexpr int NV = KDA ? 16 : 11;                 // 16-byte loads per lane and chunk
  constexpr uint32_t Tlen = NC * 64;
  const int lane = threadIdx.x & 63, lt = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bh, slice;
  const int bid = blockIdx.x;
  if (chains % 8 == 0) {                            // the kernels' XCD-aware mapping
    const int grp = bid / (8 * NS), within = bid % (8 * NS);
    bh = grp * 8 + within % 8;
    slice = within / 8;
  } else {
    bh = bid / NS;
    slice = bid % NS;
  }
  const int col0 = slice * NCOL;
  // per-chain descriptors: rows of 128 bf16 (256 B) per token, chunk images of 16 / 8 KiB
  const uint32_t row_bytes = Tlen * 256u;
  const __amdgpu_buffer_rsrc_t r0 = rsrc(t.a[0] + (size_t)bh * row_bytes, row_bytes);
  const __amdgpu_buffer_rsrc_t r1 = rsrc(t.a[1] + (size_t)bh * row_bytes, row_bytes);
  const __amdgpu_buffer_rsrc_t r2 = rsrc(t.a[2] + (size_t)bh * (KDA ? row_bytes : NC * 8192u), KDA ? row_bytes : NC * 8192u);
  const __amdgpu_buffer_rsrc_t r3 = rsrc(t.a[3] + (size_t)bh * row_bytes, row_bytes);
  const __amdgpu_buffer_rsrc_t r4 = rsrc(t.a[KDA ? 4 : 3] + (size_t)bh * (KDA ? NC * 512u : row_bytes), KDA ? NC * 512u : row_bytes);
  const __amdgpu_buffer_rsrc_t r5 = rsrc(t.a[KDA ? 5 : 3] + (size_t)bh * (KDA ? NC * 8192u : row_bytes), KDA ? NC * 8192u : row_bytes);
  const __amdgpu_buffer_rsrc_t ro = rsrc(t.o + (size_t)bh * Tlen * 512u, Tlen * 512u);
  // a slice's rows of a [T, 128] bf16 tile (v or U): NCOL * 2 bytes per row, 64 rows; lanes past
  // the tile's vectors repeat (as the kernels' loaders do)
  constexpr int VPR = NCOL / 8, VV = 64 * VPR;
  const int vu = lt % VV;
  const uint32_t tile_off = (uint32_t)(vu / VPR) * 256u + (uint32_t)col0 * 2u + (uint32_t)(vu % VPR) * 16u;

  struct Set { u32x4 v[NV]; };
  auto load = [&](Set& s, int ch) {
    if constexpr (LD) {
      const uint32_t c16 = (uint32_t)ch * 16384u, c8 = (uint32_t)ch * 8192u;
      const uint32_t lo = 16u * lane + 1024u * w;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s.v[k] = __builtin_amdgcn_raw_buffer_load_b128(r0, lo, c16 + 4096u * k, 0);
        s.v[4 + k] = __builtin_amdgcn_raw_buffer_load_b128(r1, lo, c16 + 4096u * k, 0);
      }
      if constexpr (!KDA) {
#pragma unroll
        for (int k = 0; k < 2; ++k) s.v[8 + k] = __builtin_amdgcn_raw_buffer_load_b128(r2, lo, c8 + 4096u * k, 0);
        s.v[10] = __builtin_amdgcn_raw_buffer_load_b128(r3, tile_off, (uint32_t)ch * 64u * 256u, 0);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) s.v[8 + k] = __builtin_amdgcn_raw_buffer_load_b128(r2, lo, c16 + 4096u * k, 0);
        s.v[12] = __builtin_amdgcn_raw_buffer_load_b128(r3, tile_off, (uint32_t)ch * 64u * 256u, 0);
        s.v[13] = __builtin_amdgcn_raw_buffer_load_b128(r4, 16u * (lt & 31), (uint32_t)ch * 512u, 0);
#pragma unroll
        for (int k = 0; k < 2; ++k) s.v[14 + k] = __builtin_amdgcn_raw_buffer_load_b128(r5, lo, c8 + 4096u * k, 0);
      }
    }
  };
  auto stage = [&](int buf, const Set& s) {
#pragma unroll
    for (int k = 0; k < NV; ++k) *reinterpret_cast<u32x4*>(lds[buf] + (4 * k + w) * 1024 + 16 * lane) = s.v[k];
  };
  auto ostore = [&](int ch) {
    if constexpr (ST) {
      // o[token][col0 .. col0 + NCOL) fp32: BPT bytes per token, wave w tokens 16 w ..
      constexpr int BPT = NCOL * 4, LPT = BPT / 16, TPI = 64 / LPT;
      const u32x4 val = {(uint32_t)ch, 1u, 2u, 3u};
#pragma unroll
      for (int k = 0; k < 16 / TPI; ++k) {
        const uint32_t tok = (uint32_t)ch * 64u + 16u * w + TPI * k + lane / LPT;
        __builtin_amdgcn_raw_buffer_store_b128(val, ro, tok * 512u + (uint32_t)col0 * 4u + 16u * (lane % LPT), 0,
                                               NTST ? 2 : 0);
      }
    }
  };
  uint32_t acc = 0;
  auto interval = [&](Set& ld, const Set& nx, int j) {
    load(ld, min(j + 3, STEPS - 1));
    stage((j + 1) & 1, nx);
    ostore(j);
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
    acc += lds[j & 1][(threadIdx.x * 16) % (NV * 4096)];
  };
  Set s0, s1, s2;
  load(s0, 0);
  load(s1, 1);
  load(s2, 2);
  stage(0, s0);
  __syncthreads();
  interval(s0, s1, 0);
  for (int j = 1; j + 3 < STEPS; j += 3) {
    interval(s1, s2, j);
    interval(s2, s0, j + 1);
    interval(s0, s1, j + 2);
  }
  sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

struct Buffers {
  unsigned char* src;
  unsigned char* dst;
  uint32_t* sink;
  unsigned long long* clocks;
  hipEvent_t e0, e1;
};

bool ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::printf("%s failed: %s\n", what, hipGetErrorString(e));
    return false;
  }
  return true;
}

// Best of four timed launches (after one warm-up) of one pattern; prints one line.
template <int KIB, int SH, int OB, bool NTST, bool LD>
bool run(const Buffers& b, const char* pattern, const char* what, int chain_chunks) {
  float best = 1e30f;
  for (int rep = 0; rep < 5; ++rep) {
    if (!ok(hipEventRecord(b.e0), "hipEventRecord")) return false;
    floor_kernel<KIB, SH, OB, NTST, LD><<<kGroups, 256>>>(b.src, b.dst, b.sink, b.clocks);
    if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(b.e1), "hipEventRecord") ||
        !ok(hipEventSynchronize(b.e1), "hipEventSynchronize"))
      return false;
    float ms = 0.f;
    if (!ok(hipEventElapsedTime(&ms, b.e0, b.e1), "hipEventElapsedTime")) return false;
    if (rep > 0 && ms < best) best = ms;
  }
  unsigned long long clk[2] = {0, 0};
  if (!ok(hipMemcpy(clk, b.clocks, sizeof(clk), hipMemcpyDeviceToHost), "hipMemcpy")) return false;
  const double ns = best * 1e6 / executed_steps();
  const double mhz = clk[1] ? 100.0 * (double)clk[0] / (double)clk[1] : 0.0;
  std::printf("%-12s %-14s  %2d KiB/chunk  shared by %d  o %5d B/chunk %-3s  %7.1f ns per chunk  "
              "%7.1f us per %d chunks  clock %4.0f MHz\n",
              pattern, what, KIB, SH, OB, OB ? (NTST ? "nt" : "l2") : "", ns, ns * chain_chunks / 1000.0,
              chain_chunks, mhz);
  std::fflush(stdout);
  return true;
}

// Best of four timed launches of one kernel-layout pattern; prints one line.
template <bool KDA, int NCOL, int NC, int STEPS, bool NTST, bool LD, bool ST>
bool run_layout(const Buffers& b, const Tensors& t, int chains, const char* pattern, const char* what) {
  float best = 1e30f;
  const int groups = chains * (128 / NCOL);
  for (int rep = 0; rep < 5; ++rep) {
    if (!ok(hipEventRecord(b.e0), "hipEventRecord")) return false;
    layout_kernel<KDA, NCOL, NC, STEPS, NTST, LD, ST><<<groups, 256>>>(t, b.sink, chains);
    if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(b.e1), "hipEventRecord") ||
        !ok(hipEventSynchronize(b.e1), "hipEventSynchronize"))
      return false;
    float ms = 0.f;
    if (!ok(hipEventElapsedTime(&ms, b.e0, b.e1), "hipEventElapsedTime")) return false;
    if (rep > 0 && ms < best) best = ms;
  }
  const double ns = best * 1e6 / executed_steps(STEPS);
  std::printf("%-12s %-14s  tensor layout, %2d chains x %d slices, %3d of %3d chunks  %7.1f ns per chunk  "
              "%7.1f us per %d chunks\n",
              pattern, what, chains, 128 / NCOL, STEPS, NC, ns, ns * NC / 1000.0, NC);
  std::fflush(stdout);
  return true;
}

template <bool KDA, int NCOL, int NC, int STEPS, bool NTST>
bool layout_pattern(const Buffers& b, const Tensors& t, int chains, const char* name) {
  return run_layout<KDA, NCOL, NC, STEPS, NTST, true, true>(b, t, chains, name, "loads+stores") &&
         run_layout<KDA, NCOL, NC, STEPS, NTST, true, false>(b, t, chains, name, "loads") &&
         run_layout<KDA, NCOL, NC, STEPS, NTST, false, true>(b, t, chains, name, "stores");
}

// The three stage-2 patterns: loads and o stores, the loads alone, the stores alone.
template <int KIB, int SH, int OB, bool NTST>
bool pattern(const Buffers& b, const char* name, int chain_chunks) {
  return run<KIB, SH, OB, NTST, true>(b, name, "loads+stores", chain_chunks) &&
         run<KIB, SH, 0, NTST, true>(b, name, "loads", chain_chunks) &&
         run<KIB, SH, OB, NTST, false>(b, name, "stores", chain_chunks);
}

}  // namespace

int main() {
  Buffers b{};
  const size_t src_bytes = (size_t)kMaxKiB * 1024 * kSteps * (kGroups / 4);   // SH >= 4
  const size_t dst_bytes = (size_t)8192 * kSteps * kGroups;
  if (!ok(hipMalloc(&b.src, src_bytes), "hipMalloc") || !ok(hipMalloc(&b.dst, dst_bytes), "hipMalloc") ||
      !ok(hipMalloc(&b.sink, kGroups * 256 * sizeof(uint32_t)), "hipMalloc") ||
      !ok(hipMalloc(&b.clocks, 2 * sizeof(unsigned long long)), "hipMalloc") ||
      !ok(hipMemset(b.src, 1, src_bytes), "hipMemset") || !ok(hipEventCreate(&b.e0), "hipEventCreate") ||
      !ok(hipEventCreate(&b.e1), "hipEventCreate"))
    return 1;
  // GDN headline (B4 H16 T4096): 32-column slices, k 16 + q 16 + T 8 + v 4 KiB, o 32 x 4 B per
  // token streamed past the cache.
  if (!pattern<44, 4, 8192, true>(b, "gdn_headline", 64)) return 1;
  // GDN config 4 (B1 H32 T32768): 16-column slices, k 16 + q 16 + T 8 KiB + the v tile (2 KiB,
  // loaded as 4 KiB: one 16-byte load per loader lane), o 16 x 4 B per token through the cache.
  if (!pattern<44, 8, 4096, false>(b, "gdn_config4", 512)) return 1;
  // KDA config 5 (B2 H32 T8192): 32-column slices, W, QE, KB 16 KiB each + T diag(beta) 8
  // + v 4 KiB + the decay (one 16-byte load per loader lane: 4 KiB), o streamed past the cache.
  if (!pattern<64, 4, 8192, true>(b, "kda_config5", 128)) return 1;

  // The same three in the kernels' tensor layout (one allocation per tensor, sized for the
  // largest workload: 32 chains x 32768 tokens).
  const size_t rows = (size_t)32 * 32768 * 256;           // [B*H, T, 128] bf16, 256 MiB
  unsigned char* ten[7] = {};
  const size_t sizes[7] = {rows, rows, rows, rows, (size_t)64 * 128 * 512, rows, rows * 2};
  for (int i = 0; i < 7; ++i)
    if (!ok(hipMalloc(&ten[i], sizes[i]), "hipMalloc") || !ok(hipMemset(ten[i], 1, sizes[i]), "hipMemset")) return 1;
  const Tensors t{{ten[0], ten[1], ten[2], ten[3], ten[4], ten[5]}, ten[6]};
  if (!layout_pattern<false, 32, 64, 64, true>(b, t, 64, "gdn_headline")) return 1;
  if (!layout_pattern<false, 16, 512, 96, false>(b, t, 32, "gdn_config4")) return 1;
  // config 4's pattern with the o stores non-temporal (the kernel stores them through L2)
  if (!layout_pattern<false, 16, 512, 96, true>(b, t, 32, "gdn_c4_nt")) return 1;
  if (!layout_pattern<true, 32, 128, 96, true>(b, t, 64, "kda_config5")) return 1;
  for (int i = 0; i < 7; ++i) (void)hipFree(ten[i]);
  (void)hipFree(b.src);
  (void)hipFree(b.dst);
  (void)hipFree(b.sink);
  (void)hipFree(b.clocks);
  return 0;
}
