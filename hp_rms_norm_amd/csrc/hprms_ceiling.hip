// hprms_ceiling.hip - measurement kernels of the bench library
// libhprms_bench.so (never linked into libhprms.so).  They move the bytes of
// the fused add + RMSNorm op in simpler ways, so that the op's time can be
// set beside what the same hardware needs for the same traffic:
//
//   hprms_ceil_empty     a grid of empty workgroups of 64 ... 1024 lanes
//                        (launch, dispatch and teardown of a kernel of that
//                        grid, no memory traffic)
//   hprms_ceil_read      read two tensors of n bytes (the op's two read streams)
//   hprms_ceil_write     write two tensors of n bytes (the op's two write streams)
//   hprms_ceil_copy      copy n bytes (one read and one write stream)
//   hprms_ceil_streams   the op's bytes as flat in-place or copying streams
//   hprms_ceil_flat      flat in-place streams (one or two) with a chosen
//                        workgroup shape and load order
//   hprms_ceil_skeleton  the op's own data movement in place on [rows, hidden]
//                        x and r with the lane mapping of a table row: every
//                        load first, r <- x + r stored as soon as it is formed,
//                        a row-wide reduction (DPP inside the wave, LDS and one
//                        barrier across waves), then x <- f(x, row value)
//                        stored; no fp32 arithmetic and no weight.
//
// The flat kernels give each 256-lane workgroup one 16-byte vector per lane of
// each stream (4 KiB), the shape the streamer measured fastest.  All
// accesses are non-temporal unless a kernel's flags say otherwise.  Every entry
// point returns HPRMS_OK or HPRMS_E_INVALID / HPRMS_E_LAUNCH, like the
// product's C ABI.
#include <hip/hip_runtime.h>

#include "hp_rms_norm_amd.h"
#include "hprms_device.h"

namespace hprms {
namespace {

constexpr int kFlatBlock = 256;

template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void ceil_empty_kernel() {}

// Reads vector i of a and of b; the loaded bits feed a compare whose store
// never happens for random data, so the loads cannot be dropped.
__global__ __launch_bounds__(kFlatBlock) void ceil_read_kernel(const u32x4* a, const u32x4* b, int64_t nvec,
                                                               uint32_t* sink) {
  const int64_t i = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
  if (i >= nvec) return;
  const u32x4 u = __builtin_nontemporal_load(a + i);
  const u32x4 v = __builtin_nontemporal_load(b + i);
  const uint32_t t = (u[0] ^ v[0]) + (u[1] ^ v[1]) + (u[2] ^ v[2]) + (u[3] ^ v[3]);
  if (t == 0x9e3779b9u) sink[0] = t;
}

__global__ __launch_bounds__(kFlatBlock) void ceil_write_kernel(u32x4* a, u32x4* b, int64_t nvec) {
  const int64_t i = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
  if (i >= nvec) return;
  const uint32_t v = (uint32_t)i;
  __builtin_nontemporal_store((u32x4){v, v, v, v}, a + i);
  __builtin_nontemporal_store((u32x4){~v, ~v, ~v, ~v}, b + i);
}

__global__ __launch_bounds__(kFlatBlock) void ceil_copy_kernel(u32x4* dst, const u32x4* src, int64_t nvec) {
  const int64_t i = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
  if (i >= nvec) return;
  __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// The op's bytes as flat streams of 4 KiB workgroups, to tell the number of
// streams from updating in place: kind 0 rewrites a in place (one stream, read
// then written), kind 1 rewrites a and b in place (two streams), kind 2 copies
// a and b to c and d (two read and two write streams).
template <int KIND>
__global__ __launch_bounds__(kFlatBlock) void ceil_streams_kernel(u32x4* a, u32x4* b, u32x4* c, u32x4* d,
                                                                  int64_t nvec) {
  const int64_t i = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
  if (i >= nvec) return;
  const u32x4 u = __builtin_nontemporal_load(a + i);
  if constexpr (KIND == 0) {
    __builtin_nontemporal_store(u + 1u, a + i);
  } else {
    const u32x4 v = __builtin_nontemporal_load(b + i);
    __builtin_nontemporal_store(u + v, KIND == 1 ? a + i : c + i);
    __builtin_nontemporal_store(u ^ v, KIND == 1 ? b + i : d + i);
  }
}

// The flat streams with a workgroup shape and load order of their own, to
// tell which of them the two-stream cost follows: BLOCK lanes, VPL 16-byte
// vectors per lane of each stream (lane t holds vectors t, t + BLOCK, ...),
// loads then stores as the fused op orders them (b's stores as soon as its
// sums are formed, then a's).  KIND 0 rewrites one stream `a` of 2 * VPL
// vectors per lane in place, KIND 1 rewrites `a` and `b` in place.  ORDER
// (KIND 1): 0 a and b alternating per vector, 1 all of b then all of a, 2 the
// two orders alternating per wave, 3 alternating per workgroup (consecutive
// workgroups go to different XCDs); MAP 1 / 2: the workgroups in
// xcd_xor's / xcd_runs<3>'s order.  Buffer resources span each stream
// (< 2 GiB), so the last workgroup's vectors past the end read zeros and
// drop their stores.
template <int KIND, int BLOCK, int VPL, int ORDER, int MAP = 0>
__global__ __launch_bounds__(BLOCK) void ceil_flat_kernel(uint8_t* a, uint8_t* b, uint32_t nbytes) {
  constexpr int NA = KIND == 0 ? 2 * VPL : VPL;  // vectors of `a` per lane
  const __amdgpu_buffer_rsrc_t ars = make_rsrc(a, KIND == 0 ? 2 * nbytes : nbytes);
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(b, nbytes);
  const uint32_t chunk = (uint32_t)(MAP == 1 ? xcd_xor(blockIdx.x, gridDim.x) : xcd_runs<MAP == 2 ? 3 : 0>(blockIdx.x, gridDim.x));
  const uint32_t base = (chunk * (BLOCK * NA) + threadIdx.x) * 16u;
  u32x4 u[NA], v[VPL];
  if constexpr (KIND == 0) {
#pragma unroll
    for (int k = 0; k < NA; ++k) u[k] = load16<kAuxNT>(ars, base + k * BLOCK * 16u);
#pragma unroll
    for (int k = 0; k < NA; ++k) store16<kAuxNT>(u[k] + 1u, ars, base + k * BLOCK * 16u);
  } else {
    const bool bfirst = ORDER == 1 || (ORDER == 2 && ((threadIdx.x >> 6) & 1)) || (ORDER == 3 && (blockIdx.x & 1));
    if (ORDER == 0) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        u[k] = load16<kAuxNT>(ars, base + k * BLOCK * 16u);
        v[k] = load16<kAuxNT>(brs, base + k * BLOCK * 16u);
      }
    } else if (bfirst) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) v[k] = load16<kAuxNT>(brs, base + k * BLOCK * 16u);
#pragma unroll
      for (int k = 0; k < VPL; ++k) u[k] = load16<kAuxNT>(ars, base + k * BLOCK * 16u);
    } else {
#pragma unroll
      for (int k = 0; k < VPL; ++k) u[k] = load16<kAuxNT>(ars, base + k * BLOCK * 16u);
#pragma unroll
      for (int k = 0; k < VPL; ++k) v[k] = load16<kAuxNT>(brs, base + k * BLOCK * 16u);
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) store16<kAuxNT>(u[k] + v[k], brs, base + k * BLOCK * 16u);
#pragma unroll
    for (int k = 0; k < VPL; ++k) store16<kAuxNT>(u[k] ^ v[k], ars, base + k * BLOCK * 16u);
  }
}

typedef void (*flat_fn)(uint8_t*, uint8_t*, uint32_t);
struct FlatEntry {
  int kind, block, vpl, order, map;
  flat_fn fn;
};
#define HPRMS_FLAT(KIND, BLOCK, VPL, ORDER) {KIND, BLOCK, VPL, ORDER, 0, &ceil_flat_kernel<KIND, BLOCK, VPL, ORDER>},
#define HPRMS_FLAT_MAPPED(KIND, BLOCK, VPL, MAP) \
  {KIND, BLOCK, VPL, 0, MAP, &ceil_flat_kernel<KIND, BLOCK, VPL, 0, MAP>},
#define HPRMS_FLAT_ORDERS(BLOCK, VPL) \
  HPRMS_FLAT(0, BLOCK, VPL, 0) HPRMS_FLAT(1, BLOCK, VPL, 0) HPRMS_FLAT(1, BLOCK, VPL, 1) \
  HPRMS_FLAT(1, BLOCK, VPL, 2) HPRMS_FLAT(1, BLOCK, VPL, 3)
// the workgroup orders of xcd_xor (map 1) and xcd_runs<3> (map 2) for one and two streams
#define HPRMS_FLAT_MAPS(BLOCK, VPL) \
  HPRMS_FLAT_MAPPED(0, BLOCK, VPL, 1) HPRMS_FLAT_MAPPED(0, BLOCK, VPL, 2) HPRMS_FLAT_MAPPED(1, BLOCK, VPL, 1) \
  HPRMS_FLAT_MAPPED(1, BLOCK, VPL, 2)
const FlatEntry kFlat[] = {
    HPRMS_FLAT_ORDERS(64, 1) HPRMS_FLAT_ORDERS(128, 1) HPRMS_FLAT_ORDERS(256, 1) HPRMS_FLAT_ORDERS(512, 1)
    HPRMS_FLAT_ORDERS(1024, 1) HPRMS_FLAT_ORDERS(256, 2) HPRMS_FLAT_ORDERS(512, 2) HPRMS_FLAT_ORDERS(1024, 2)
    HPRMS_FLAT_ORDERS(256, 4) HPRMS_FLAT_ORDERS(1024, 4)
    HPRMS_FLAT_MAPS(256, 1) HPRMS_FLAT_MAPS(512, 1) HPRMS_FLAT_MAPS(1024, 1) HPRMS_FLAT_MAPS(256, 2)
    HPRMS_FLAT_MAPS(1024, 4)
};

struct SkelArgs {
  uint16_t* x;
  uint16_t* r;
  int64_t rows;
  int32_t hidden;
  int32_t nvec;
};

// The op's data movement with a table row's shape (LPR lanes per row, VPL
// vectors per lane, BLOCK lanes per workgroup) and cache-policy flags (bits
// 0, 1, 3, 4 and 7 as in fused_vec_kernel).  Contiguous rows, hidden % 8 == 0,
// 16-byte aligned tensors.
template <int LPR, int VPL, int BLOCK, int FLAGS>
__global__ __launch_bounds__(BLOCK) void ceil_skeleton_kernel(SkelArgs a) {
  constexpr int RPB = BLOCK / LPR;
  constexpr int GW = LPR < 64 ? LPR : 64;
  constexpr int WPR = LPR > 64 ? LPR / 64 : 1;
  constexpr int NW = BLOCK / 64;
  constexpr int LAUX = ((FLAGS & 1) ? kAuxNT : 0) | ((FLAGS & 8) ? kAuxSC1 : 0);
  constexpr int SAUX = ((FLAGS & 2) ? kAuxNT : 0) | ((FLAGS & 16) ? kAuxSC1 : 0);
  constexpr uint32_t CH = LPR * 16;
  __shared__ float red[WPR > 1 ? NW : 1];

  const int tid = threadIdx.x;
  const int lane = tid & (LPR - 1);
  const int rib = tid / LPR;
  const int64_t row0 = (int64_t)blockIdx.x * RPB;
  const int64_t left = a.rows - row0;
  const int nrows = left < RPB ? (int)left : RPB;
  const bool row_ok = rib < nrows;
  const uint32_t bytes = (uint32_t)((int64_t)nrows * a.hidden * 2);
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x + row0 * a.hidden, bytes);
  const __amdgpu_buffer_rsrc_t rrs = make_rsrc(a.r + row0 * a.hidden, bytes);
  const uint32_t off = (uint32_t)rib * (uint32_t)a.hidden * 2u + (uint32_t)lane * 16u;

  u32x4 xv[VPL], rv[VPL];
  uint32_t o[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) o[k] = (row_ok && (k * LPR + lane) < a.nvec) ? off + k * CH : kOOB;
  if constexpr ((FLAGS & 128) != 0) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) rv[k] = load16<LAUX>(rrs, o[k]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < VPL; ++k) xv[k] = load16<LAUX>(xrs, o[k]);
    __builtin_amdgcn_sched_barrier(0);
  } else {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      xv[k] = load16<LAUX>(xrs, o[k]);
      rv[k] = load16<LAUX>(rrs, o[k]);
    }
  }
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    u32x4 s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[j] = xv[k][j] + rv[k][j];
      acc += s[j] & 0xffu;
    }
    rv[k] = s;
    store16<SAUX>(s, rrs, o[k]);
  }
  float tot = group_sum<GW>((float)acc);
  if constexpr (WPR > 1) {
    const int wave = tid >> 6;
    if ((tid & 63) == 0) red[wave] = tot;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    tot = red[w0];
#pragma unroll
    for (int j = 1; j < WPR; ++j) tot += red[w0 + j];
  }
  const uint32_t t = __float_as_uint(tot);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = xv[k][j] ^ (rv[k][j] + t);
    store16<SAUX>(v, xrs, o[k]);
  }
}

typedef void (*skel_fn)(SkelArgs);
struct SkelEntry {
  int lpr, vpl, block, flags;
  skel_fn fn;
};

#define HPRMS_SKEL(LPR, VPL, BLOCK, FLAGS) {LPR, VPL, BLOCK, FLAGS, &ceil_skeleton_kernel<LPR, VPL, BLOCK, FLAGS>},
#define HPRMS_SKEL_FLAGS(LPR, VPL, BLOCK) \
  HPRMS_SKEL(LPR, VPL, BLOCK, 3) HPRMS_SKEL(LPR, VPL, BLOCK, 27) HPRMS_SKEL(LPR, VPL, BLOCK, 131) \
  HPRMS_SKEL(LPR, VPL, BLOCK, 155)

// the lane shapes of the bandwidth table's rows and their neighbours
const SkelEntry kSkel[] = {
    HPRMS_SKEL_FLAGS(32, 4, 256) HPRMS_SKEL_FLAGS(64, 4, 256) HPRMS_SKEL_FLAGS(128, 3, 256)
    HPRMS_SKEL_FLAGS(128, 4, 256) HPRMS_SKEL_FLAGS(256, 2, 256) HPRMS_SKEL_FLAGS(256, 4, 256)
    HPRMS_SKEL_FLAGS(512, 2, 512) HPRMS_SKEL_FLAGS(512, 3, 512) HPRMS_SKEL_FLAGS(512, 4, 512)
    HPRMS_SKEL_FLAGS(1024, 2, 1024) HPRMS_SKEL_FLAGS(256, 8, 256) HPRMS_SKEL_FLAGS(1024, 3, 1024)
    HPRMS_SKEL_FLAGS(1024, 4, 1024) HPRMS_SKEL_FLAGS(32, 8, 64) HPRMS_SKEL_FLAGS(32, 12, 64)
    // the other splits of a 512-vector row (H = 4096), one to eight rows per workgroup
    HPRMS_SKEL(64, 8, 64, 131) HPRMS_SKEL(64, 8, 128, 131) HPRMS_SKEL(64, 8, 256, 131) HPRMS_SKEL(64, 8, 512, 131)
    HPRMS_SKEL(128, 4, 128, 131) HPRMS_SKEL(128, 4, 512, 131) HPRMS_SKEL(256, 2, 512, 131)
    HPRMS_SKEL(512, 1, 512, 131)
};

int launched() { return hipGetLastError() == hipSuccess ? HPRMS_OK : HPRMS_E_LAUNCH; }

int64_t flat_grid(int64_t nvec) { return (nvec + kFlatBlock - 1) / kFlatBlock; }

bool flat_ok(const void* p, int64_t nbytes) {
  return p && ((uintptr_t)p & 15u) == 0 && nbytes > 0 && nbytes % 16 == 0 && flat_grid(nbytes / 16) <= 0x7fffffff;
}

}  // namespace
}  // namespace hprms

using namespace hprms;

extern "C" {

// block: 64, 128, 256, 512 or 1024 lanes (the workgroup sizes of the table and the fill map)
int hprms_ceil_empty(int64_t grid, int block, hipStream_t stream) {
  if (grid < 1 || grid > 0x7fffffff) return HPRMS_E_INVALID;
  const dim3 g((unsigned)grid);
  if (block == 64)
    ceil_empty_kernel<64><<<g, dim3(64), 0, stream>>>();
  else if (block == 128)
    ceil_empty_kernel<128><<<g, dim3(128), 0, stream>>>();
  else if (block == 256)
    ceil_empty_kernel<256><<<g, dim3(256), 0, stream>>>();
  else if (block == 512)
    ceil_empty_kernel<512><<<g, dim3(512), 0, stream>>>();
  else if (block == 1024)
    ceil_empty_kernel<1024><<<g, dim3(1024), 0, stream>>>();
  else
    return HPRMS_E_INVALID;
  return launched();
}

int hprms_ceil_read(const void* a, const void* b, int64_t nbytes, void* sink, hipStream_t stream) {
  if (!flat_ok(a, nbytes) || !flat_ok(b, nbytes) || !sink) return HPRMS_E_INVALID;
  const int64_t nvec = nbytes / 16;
  ceil_read_kernel<<<dim3((unsigned)flat_grid(nvec)), dim3(kFlatBlock), 0, stream>>>(
      (const u32x4*)a, (const u32x4*)b, nvec, (uint32_t*)sink);
  return launched();
}

int hprms_ceil_write(void* a, void* b, int64_t nbytes, hipStream_t stream) {
  if (!flat_ok(a, nbytes) || !flat_ok(b, nbytes)) return HPRMS_E_INVALID;
  const int64_t nvec = nbytes / 16;
  ceil_write_kernel<<<dim3((unsigned)flat_grid(nvec)), dim3(kFlatBlock), 0, stream>>>((u32x4*)a, (u32x4*)b, nvec);
  return launched();
}

int hprms_ceil_copy(void* dst, const void* src, int64_t nbytes, hipStream_t stream) {
  if (!flat_ok(dst, nbytes) || !flat_ok(src, nbytes)) return HPRMS_E_INVALID;
  const int64_t nvec = nbytes / 16;
  ceil_copy_kernel<<<dim3((unsigned)flat_grid(nvec)), dim3(kFlatBlock), 0, stream>>>((u32x4*)dst,
                                                                                   (const u32x4*)src, nvec);
  return launched();
}

// kind 0: a (2 * nbytes) rewritten in place; kind 1: a and b (nbytes each)
// rewritten in place; kind 2: a and b copied to c and d (nbytes each).
int hprms_ceil_streams(int kind, void* a, void* b, void* c, void* d, int64_t nbytes, hipStream_t stream) {
  if (kind < 0 || kind > 2 || !flat_ok(a, kind == 0 ? 2 * nbytes : nbytes)) return HPRMS_E_INVALID;
  if (kind >= 1 && !flat_ok(b, nbytes)) return HPRMS_E_INVALID;
  if (kind == 2 && (!flat_ok(c, nbytes) || !flat_ok(d, nbytes))) return HPRMS_E_INVALID;
  const int64_t nvec = (kind == 0 ? 2 * nbytes : nbytes) / 16;
  const dim3 g((unsigned)flat_grid(nvec));
  u32x4 *pa = (u32x4*)a, *pb = (u32x4*)b, *pc = (u32x4*)c, *pd = (u32x4*)d;
  if (kind == 0)
    ceil_streams_kernel<0><<<g, dim3(kFlatBlock), 0, stream>>>(pa, pb, pc, pd, nvec);
  else if (kind == 1)
    ceil_streams_kernel<1><<<g, dim3(kFlatBlock), 0, stream>>>(pa, pb, pc, pd, nvec);
  else
    ceil_streams_kernel<2><<<g, dim3(kFlatBlock), 0, stream>>>(pa, pb, pc, pd, nvec);
  return launched();
}

// kind 0: a (2 * nbytes) rewritten in place; kind 1: a and b (nbytes each)
// rewritten in place; block lanes x vpl vectors per lane per stream, load
// order `order` (ceil_flat_kernel).  nbytes % 16 == 0, below 1 GiB.
// order 4 / 5: alternating loads (order 0) with the workgroups in xcd_xor's
// order / in xcd_runs<3>'s (for kind 0 too).
int hprms_ceil_flat(int kind, int block, int vpl, int order, void* a, void* b, int64_t nbytes, hipStream_t stream) {
  if (!flat_ok(a, nbytes) || (kind == 1 && !flat_ok(b, nbytes)) || nbytes >= (int64_t(1) << 30))
    return HPRMS_E_INVALID;
  const int map = order >= 4 ? order - 3 : 0;
  const int ord = order >= 4 || kind == 0 ? 0 : order;
  for (const FlatEntry& e : kFlat) {
    if (e.kind != kind || e.block != block || e.vpl != vpl || e.order != ord || e.map != map) continue;
    const int64_t per_wg = (int64_t)block * vpl * 16;  // bytes of each stream per workgroup (kind 0: of half `a`)
    const int64_t grid = (nbytes + per_wg - 1) / per_wg;
    hipLaunchKernelGGL(e.fn, dim3((unsigned)grid), dim3(block), 0, stream, (uint8_t*)a,
                       (uint8_t*)(kind == 0 ? a : b), (uint32_t)nbytes);
    return launched();
  }
  return HPRMS_E_INVALID;
}

// x and r: contiguous [rows, hidden] 16-bit tensors, 16-byte aligned, hidden %
// 8 == 0, lpr * vpl * 8 >= hidden and a row group within 2 GiB.  (lpr, vpl,
// block, flags) must be one of kSkel's shapes.
int hprms_ceil_skeleton(void* x, void* r, int64_t rows, int64_t hidden, int lpr, int vpl, int block, int flags,
                        hipStream_t stream) {
  if (!x || !r || ((uintptr_t)x & 15u) || ((uintptr_t)r & 15u) || rows < 1 || hidden < 8 || hidden % 8 != 0 ||
      (int64_t)lpr * vpl * 8 < hidden)
    return HPRMS_E_INVALID;
  for (const SkelEntry& e : kSkel) {
    if (e.lpr != lpr || e.vpl != vpl || e.block != block || e.flags != flags) continue;
    const int64_t rpb = block / lpr;
    if (rpb * hidden * 2 >= (int64_t)kOOB) return HPRMS_E_INVALID;
    const int64_t grid = (rows + rpb - 1) / rpb;
    if (grid > 0x7fffffff) return HPRMS_E_INVALID;
    SkelArgs a{(uint16_t*)x, (uint16_t*)r, rows, (int32_t)hidden, (int32_t)(hidden / 8)};
    hipLaunchKernelGGL(e.fn, dim3((unsigned)grid), dim3(block), 0, stream, a);
    return launched();
  }
  return HPRMS_E_INVALID;
}

}  // extern "C"
