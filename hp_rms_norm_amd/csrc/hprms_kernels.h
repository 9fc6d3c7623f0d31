// hprms_kernels.h - the gfx950 kernels of libhprms.so.
//
// Fused residual-add + RMSNorm, "vector" tiers (hidden >= 8; rows at any
// 2-byte boundary, see FLAGS bits 5 and 6 below).  A row of H elements is
// nvec = H/8 whole 16-byte vectors (plus a tail when H % 8 != 0, and a head
// when the tail variant shifts the row).  A
// workgroup of BLOCK lanes works on RPB = BLOCK/LPR rows at a time, LPR lanes
// per row; lane l of a row owns vectors l, l+LPR, ..., l+(VPL-1)*LPR, so every
// load instruction of a wave covers 1 KiB of contiguous bytes.  The row is
// read from HBM once: the rounded sum stays on the CU (VPL-LDSV vectors in
// VGPRs, LDSV vectors in per-lane LDS slots) until the output is written.
//
//   per row:  load x, r (16 B each per vector)          global -> VGPR
//             s = rne(x + r); store s to residual; ss += s^2 (fp32)
//             row sum of ss: DPP/swizzle inside the wave, then one LDS
//             exchange + barrier when the row spans several waves
//             inv = 1 / sqrt(ss / H + eps)
//             out = rne((s * inv) * w); store out to input
//
// The weight vectors a lane needs are re-read per row group (they stay hot in
// L2): either together with the row (WLATE = 0) or after the residual has
// been stored (WLATE = 1), when the residual registers are free again, which
// keeps the peak VGPR count low enough for 8 waves per SIMD at VPL = 4.
//
// FLAGS bit 0 marks the row loads non-temporal, bit 1 the stores: the rows
// are touched once, so they should not displace the weight from the caches.
// Bits 3 and 4 add the sc1 (device-scope) policy bit to the loads and to the
// stores respectively; bit 13 (bench library) adds sc0 to the stores.  Bit 5
// marks the variants for rows that are not 128-byte aligned (the host sends
// them there; the code is correct for rows at any 2-byte boundary: 16-byte
// accesses at unaligned addresses are legal on gfx9-family GPUs under the ROCm
// runtime, which runs them in unaligned mode, and hipcc relies on the same for
// ordinary code).  In modes 0, 1, 3 and 4 these variants also rotate each
// row's lane mapping: with the row's first body vector rp 16-byte steps past a
// 512-byte boundary of the rotation stream (`phases`, below; a 16 * LPR-byte
// boundary for LPR < 32; rp = 0 when that phase is not a multiple of 16
// bytes), slot k * LPR + lane holds body vector k * LPR + lane - rp and the
// first rp slots the row's last rp vectors, so every wave's 1 KiB access
// starts on a 512-byte boundary and writes whole cache lines (lines written
// in two parts by two accesses cost 9-13% at a 16-byte offset; 512-byte
// boundaries rather than 128-byte ones measured up to 1% faster at 16K-32K).
// The phase depends on a buffer's address only modulo 512 bytes, which
// torch's allocator fixes, so the result's bits (the lanes' summation order)
// do not depend on where a buffer was allocated.
// Bit 6 selects the tail variant (TAIL), for widths that are not a multiple
// of 8 (hidden >= 8) and for shifted rows (hidden >= 16).  Row r is shifted by
// delta = (shift base + r * shift step) mod 8 elements (`phases`; both 0: no shift): the
// lanes' "body" vectors start at element 8j - delta (j >= 1 when delta > 0),
// so a stream whose row r starts delta elements past a vector boundary (16
// bytes; 8 bytes for the FP8 output) is accessed aligned; the elements before the first body
// vector come from a head vector (the row's first 16 bytes, lane 0) and those
// after the last from a tail vector (the row's last 16 bytes, the lane holding
// the last body vector, or lane 1 when that is lane 0).  An edge vector counts
// only its elements no body vector holds, and stores all 8: the others equal
// what their body vector stores, from a lane of the same wave, and a wave
// issues all its loads before its stores.  Bit 7 issues all
// of a lane's residual loads before its input loads (otherwise the two
// streams alternate per vector); which is faster depends on the shape.
// Bit 14 (tail variants with the late weight and rows of several waves, not
// the FP8 output): a shifted row reads its weight 2 * delta bytes off the
// weight's 16-byte vectors, and such loads cost the L1 path.  With the bit the
// workgroup loads the whole weight once, aligned, before its first row
// group's loads, writes it to LDS after them, and every row reads its
// vectors from there (five dwords each, funnel-shifted by the row's 2-byte
// phase) after the row-sum barrier.  Bit 15 (MODE 4): each group of vectors
// loads every part before adding the first (the latency rows).  Bits 16-18
// (V > 0): workgroup g takes row group xcd_runs<V>(g) rather than g, so each
// XCD works on runs of 2^V consecutive row groups (hprms_device.h).
//
// The residual is stored as soon as it is formed: deferring it to the output
// phase (one write burst per workgroup) measured up to 5% slower.
//
// MODE 0 is the fused op (in place on input and residual); MODE 1 is the
// plain RMSNorm (reads `input`, writes `out`, no residual stream); MODE 2 is
// the fused op with an FP8 output: the 16-bit output y is quantised per row
// (scale = max(amax|y| / 448, FLT_MIN) to scale[row], q = e4m3fn(clamp(y *
// (1 / scale))) to q), or, with FusedArgs::static_scale set, with that one
// given scale for every row (no row maximum, no scale written); the residual
// is updated in place and `input` is only read.
// The row maximum is a second DPP/LDS reduction over the 16-bit magnitudes
// (sign-magnitude bit patterns order like their values, NaN above inf).
// MODE 3 is the fused op out of place: input and residual are only read, the
// sum goes to res_out and the output to out.  MODE 4 adds nparts partial rows
// first (the buffers of a tensor-parallel all-reduce): a = rne(p0 + p1 + ...)
// summed in fp32 left to right and rounded once, then the fused op on a, with
// the residual updated in place and the output written to out.  MODES 5 and 6
// are the fused op with an OCP MX output (MXFP8 / MXFP4): the 16-bit output y
// is cut into blocks of 32 consecutive elements -- the 8 elements of four
// adjacent lanes at one vector index, so a block's maximum is one DPP quad
// reduction -- each with the scale 2^s, s = floor(log2 max|y|) - emax (8 for
// E4M3, 2 for E2M1) clamped to [-127, 127], written as one E8M0 byte, and
// elements y / 2^s rounded to nearest even and saturated (E4M3 bytes; E2M1
// codes two per byte, the even element in the low nibble; both conversions
// are gfx950 instructions).  A block holding NaN or infinity gets the scale
// byte 0xFF and unscaled elements.  The
// residual is updated in place and `input` is only read, as in MODE 2.
// MODE 7 is the fused op with an FP8 (e4m3fn) output and one float32 scale
// per 128 consecutive elements of a row (the 16 adjacent lanes of a DPP row
// at one vector index, so a group's maximum is one 16-lane DPP reduction):
// scale = max(amax|y| / 448, FLT_MIN) and q = e4m3fn(clamp(y * (1 / scale)))
// per group, as MODE 2 per row.  The scales sit at a row stride and a group
// stride of their own, so rows of scales and the column-major (token-minor)
// layout of block-scaled GEMMs are written alike.
#pragma once

#include "hprms_device.h"

namespace hprms {

// The kernel's arguments.  Everything the in-place op and the plain RMSNorm
// (MODES 0 and 1) read comes first, as scalar arguments (fused_vec_kernel's
// x_rows ... eps, 14 dwords): hipcc's -amdgpu-kernarg-preload-count has gfx950
// preload up to the first 14 dwords of the argument block into SGPRs at wave
// launch, so their first row loads wait for no scalar memory load (the
// compiler waits for every scalar load the row loop uses before the loop's
// first iteration; a copy kernel measured 0.2 us less per launch at 16-256 MB
// with its arguments preloaded; a by-value struct is never preloaded).  The
// row strides are 32-bit (the host sends larger strides to the general
// kernel); the off-grid variants' per-row phases take one dword:
//   bits 0-9   rotation (FLAGS bit 5, modes 0, 1, 3, 4): the rotation
//   bits 10-19 stream's row r starts (base + r * step) mod 512 bytes past a
//              512-byte boundary (both < 512; both 0: no rotation)
//   bits 20-22 shift (FLAGS bit 6): row r is shifted by (base + r * step)
//   bits 24-26 mod 8 elements (both 0: no shift)
__host__ __device__ constexpr uint32_t pack_phases(uint32_t rot_base, uint32_t rot_step, uint32_t shift_base,
                                                   uint32_t shift_step) {
  return (rot_base & 1023u) | (rot_step & 1023u) << 10 | (shift_base & 7u) << 20 | (shift_step & 7u) << 24;
}

// FusedArgs holds the rest:
struct FusedArgs {
  uint16_t* out;         // 16-bit output rows (MODES 1, 3, 4; MODE 0: == x)
  int64_t out_stride;
  uint8_t* q;            // MODES 2, 5, 6: quantised output rows
  float* scale;          // MODE 2: per-row scales
  const float* static_scale;  // MODE 2: one scale for every row, given (null: per-row scales, written)
  const float* scale_ub;      // MODE 2, per-row scales: upper bound on the row maximum (null: none)
  int64_t q_stride;      // MODES 2, 5, 6: bytes between quantised rows
  uint16_t* res_out;     // MODE 3: residual output rows
  int64_t res_out_stride;
  int32_t nparts;        // MODE 4: number of partial rows summed (x_rows is part 0)
  const uint16_t* parts[HPRMS_MAX_PARTS];  // MODE 4: parts[g] has row stride x_stride
  uint8_t* mx_scale;     // MODES 5, 6: E8M0 scale bytes; MODE 7: float32 scales (hidden / 32 bytes per row)
  int64_t mx_scale_stride;  // bytes between scale rows
  int64_t mx_group_stride;  // MODE 7: bytes between a row's consecutive scales (4: rows of scales)
  int64_t* timeline;     // FLAGS bit 9 only (bench library): 4 values per workgroup
};

// Waves per SIMD the compiler must leave room for: the tail variant of the
// 1024-lane shapes with up to 2 vectors per lane is held to 64 VGPRs, so two
// workgroups share a CU as they do without the tail (the FP8 form needed 66:
// held to 64 it runs 19-23% faster at 13K-16K).  At 3 vectors per lane the
// same limit spills and measured 3-7% slower.  FLAGS bit 8 asks for 8 waves
// per SIMD (64 VGPRs) on any shape.
template <int FLAGS, int BLOCK, int VPL>
constexpr int kMinWavesPerEU = ((FLAGS & 256) != 0 || ((FLAGS & 64) != 0 && BLOCK == 1024 && VPL <= 2)) ? 8 : 1;

template <int DT, int MODE, int LPR, int VPL, int LDSV, int BLOCK, int FLAGS, int WLATE>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(kMinWavesPerEU<FLAGS, BLOCK, VPL>)))
void fused_vec_kernel(const uint16_t* x_rows,  // input rows (MODE 0: also the output; MODE 4: part 0)
                      uint16_t* res_rows,      // residual rows (MODE 1: the output rows)
                      const uint16_t* w,       // weight [hidden]
                      int64_t rows,
                      int32_t x_stride, int32_t res_stride,  // elements
                      int32_t hidden,
                      int32_t grid,            // workgroups launched (<= ceil(rows / RPB))
                      uint32_t phases,         // off-grid variants: rotation and shift (pack_phases)
                      float eps,
                      FusedArgs a) {
  const int32_t nvec = hidden >> 3;  // whole 16-byte vectors per row
  static_assert(LPR >= 16 && (LPR & (LPR - 1)) == 0 && BLOCK % LPR == 0 && BLOCK % 64 == 0, "shape");
  static_assert(LDSV >= 0 && LDSV <= VPL, "LDS share");
  using F = Fmt<DT>;
  constexpr int RPB = BLOCK / LPR;
  constexpr int GW = LPR < 64 ? LPR : 64;
  constexpr int WPR = LPR > 64 ? LPR / 64 : 1;
  constexpr int NW = BLOCK / 64;
  constexpr int VREG = VPL - LDSV;
  static_assert(MODE >= 0 && MODE <= 7, "mode");
  constexpr bool RES = MODE != 1;                                  // residual stream read
  constexpr bool MX = MODE == 5 || MODE == 6;                      // OCP MX output
  constexpr bool GQ = MODE == 7;                                   // FP8, one scale per 128 elements
  constexpr bool BLOCKQ = MX || GQ;                                // per-block scales from DPP maxima
  static_assert(!GQ || LPR % 16 == 0, "a 128-element group is 16 adjacent lanes' vectors");
  constexpr bool OUT16 = MODE == 1 || MODE == 3 || MODE == 4;      // 16-bit output to `out`
  constexpr bool TAIL = (FLAGS & 64) != 0 && !BLOCKQ;              // shifted rows, head and tail vectors
  // rows off the 128-byte grid: each row's lane mapping rotated so that every
  // wave's 1 KiB access starts on a 512-byte boundary (`phases` bits 0-19)
  // (not the FP8 and block-scaled outputs: the FP8 form's 1024 x 2 tail
  // kernel, held to 64 VGPRs, would spill, and a block must stay one group
  // of adjacent lanes)
  constexpr bool ROT = (FLAGS & 32) != 0 && !BLOCKQ && MODE != 2;
  // residual loads issued first (not for the partial-sum form, where it measured 0.1-1.8% slower)
  constexpr bool RFIRST = (FLAGS & 128) != 0 && RES && MODE != 4;
  // FLAGS bit 20 / bit 21 (bench library, with bit 7): the residual-first and
  // input-first orders alternating per wave / per workgroup (consecutive
  // workgroups run on different XCDs)
  constexpr bool ALTW = RFIRST && (FLAGS & 1048576) != 0;
  constexpr bool ALTG = RFIRST && (FLAGS & 2097152) != 0;
  constexpr int LAUX = ((FLAGS & 1) ? kAuxNT : 0) | ((FLAGS & 8) ? kAuxSC1 : 0);
  constexpr int SAUX = ((FLAGS & 2) ? kAuxNT : 0) | ((FLAGS & 16) ? kAuxSC1 : 0) | ((FLAGS & 8192) ? kAuxSC0 : 0);
  // FLAGS bits 22-25 (bench library): one stream's accesses without the
  // policy bits the others keep: the input's loads (22) or the residual's
  // (23) without nt and sc1, the residual's stores (24) or the output's (25)
  // without nt
  constexpr int XLAUX = (FLAGS & 4194304) ? 0 : LAUX;
  constexpr int RLAUX = (FLAGS & 8388608) ? 0 : LAUX;
  constexpr int RSAUX = (FLAGS & 16777216) ? (SAUX & ~kAuxNT) : SAUX;
  constexpr int OSAUX = (FLAGS & 33554432) ? (SAUX & ~kAuxNT) : SAUX;
  constexpr uint32_t CH = LPR * 16;  // byte distance between a lane's vectors
  // FLAGS bit 10 (bench library): row groups in xcd_xor's order; bits 16-18,
  // V > 0: in xcd_runs<V>'s order (runs of 2^V row groups per XCD; the table
  // takes it for the in-place op at two row pitches, the bench library for
  // its sweeps)
  constexpr bool WXOR = (FLAGS & 1024) != 0;
  constexpr int WRUNS = (FLAGS >> 16) & 7;
  // The output phase's unpack of the held row.  With the square phase's lo /
  // hi the compiler merges the two and keeps the row's unpacked floats live
  // across the reduction (more VGPRs); FLAGS bit 12 (bench library) unpacks
  // through a byte permute instead (Fmt::olo / ohi), which keeps packed words
  // and lowers VGPRs and raises occupancy, but measured 0-3% slower (2.5-3.2%
  // at 28K-32K, 2.9% at 16K): more rows in flight per CU do not stream faster.
  auto olo = [](uint32_t w) { if constexpr ((FLAGS & 4096) != 0) return F::olo(w); else return F::lo(w); };
  auto ohi = [](uint32_t w) { if constexpr ((FLAGS & 4096) != 0) return F::ohi(w); else return F::hi(w); };

  __shared__ float red[2][WPR > 1 ? NW : 1];
  __shared__ u32x4 spill[LDSV > 0 ? LDSV * BLOCK : 1];
  // WLDS: the weight staged in LDS (FLAGS bit 14): the row's whole vectors,
  // its partial last vector and one vector of slack for the five-dword reads
  constexpr bool WLDS = (FLAGS & 16384) != 0;
  static_assert(!WLDS || (TAIL && WLATE && LDSV == 0 && WPR > 1 && MODE != 2), "weight staged in LDS");
  static_assert((FLAGS & 32768) == 0 || MODE == 4, "parts prefetched: partial sums only");
  constexpr int NST = WLDS ? (LPR * VPL + BLOCK - 1) / BLOCK : 1;  // staged vectors per thread
  __shared__ u32x4 wlds[WLDS ? LPR * VPL + 2 : 1];
  bool staged = false;

  const int tid = threadIdx.x;
  const int lane = tid & (LPR - 1);
  const int rib = tid / LPR;
  const int wave = tid >> 6;
  // FLAGS bit 9 (bench library only): per workgroup, the realtime clock
  // (100 MHz) at its start and after its last store has completed, and the
  // hardware ids of the CU it ran on
  constexpr bool TIMELINE = (FLAGS & 512) != 0;
  const uint64_t t_start = TIMELINE ? __builtin_amdgcn_s_memrealtime() : 0;

  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, (uint32_t)hidden * 2u);

  // slots past the row's vectors: their row accesses and (in the tail
  // variant, whose shifted weight slot past the row could start inside the
  // weight) their weight loads take the out-of-range offset; elsewhere such a
  // weight slot starts at or past the weight's end and the range check
  // returns zeros
  bool vec_ok[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) vec_ok[k] = (k * LPR + lane) < nvec;

  int buf = 0;
  // the grid never exceeds the row group count, so every workgroup has a
  // first row group
  const int64_t ngroups = (rows + RPB - 1) / RPB;
  // hidden as binary32 (exact: 1 <= hidden < 2^24), built with integer
  // operations so that it stays in an SGPR (a conversion would take a VGPR)
  const uint32_t hb = (uint32_t)hidden;
  const int he = 31 - __builtin_clz(hb);
  const float hidden_f = __builtin_bit_cast(float, (uint32_t)(127 + he) << 23 | ((hb << (23 - he)) & 0x7fffffu));
  for (int64_t g = blockIdx.x;;) {
    const int64_t row0 = (WXOR ? xcd_xor(g, ngroups) : xcd_runs<WRUNS>(g, ngroups)) * RPB;
    const int64_t left = rows - row0;
    const int nrows = left < RPB ? (int)left : RPB;
    const bool row_ok = rib < nrows;

    // TAIL: this row's shift delta (elements), its first body vector j0 and
    // its body vectors nb; without the tail every row is nvec whole vectors
    int delta = 0, j0 = 0, nb = nvec, t = 0;
    uint32_t wshift = 0;
    if constexpr (TAIL) {
      delta = (int)((((phases >> 20) & 7u) + (uint32_t)(row0 + rib) * (phases >> 24)) & 7u);
      j0 = delta > 0 ? 1 : 0;
      const int jend = (hidden + delta) >> 3;
      nb = jend - j0;  // >= 1: hidden >= 8, and >= 16 when shifted
      t = hidden + delta - 8 * jend;  // elements after the last body vector
      wshift = 16u * (uint32_t)j0 - 2u * (uint32_t)delta;
    }
    // ROT: the row's rotation rp, in vectors, from the phase of its first
    // body vector in the rotation stream modulo RG bytes (when that is a
    // multiple of 16 bytes); slot k * LPR + lane then holds body vector
    // k * LPR + lane - rp, and the first rp slots (k = 0, lane < rp < LPR)
    // the row's last rp vectors
    int rp = 0;
    if constexpr (ROT) {
      constexpr uint32_t RG = LPR * 16 < 512 ? LPR * 16 : 512;
      const uint32_t ph = ((phases & 1023u) + (uint32_t)(row0 + rib) * ((phases >> 10) & 1023u) + wshift) & (RG - 1);
      if ((ph & 15u) == 0 && nb >= (int)(RG / 16)) rp = (int)(ph >> 4);
    }
    const uint32_t lofs = (uint32_t)(lane - rp) * 16u;        // lane * 16 without rotation
    const uint32_t wrap = (ROT && lane < rp) ? (uint32_t)nb : 0u;  // vectors added to slot k = 0
    // byte offset of slot k's vector past the lane's first (16-byte vectors)
    auto vk = [&](int k) -> uint32_t { return (uint32_t)(k * CH) + (k == 0 ? wrap * 16u : 0u); };

    const uint32_t xbytes = (uint32_t)(((int64_t)(nrows - 1) * x_stride + hidden) * 2);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x_rows + row0 * x_stride, xbytes);
    uint32_t xoff = (uint32_t)rib * (uint32_t)x_stride * 2u + lofs;

    // rrs/roff: residual loads (the stores' resources come after the loads)
    __amdgpu_buffer_rsrc_t rrs = xrs;
    uint32_t roff = 0;
    if constexpr (RES) {
      const uint32_t rbytes = (uint32_t)(((int64_t)(nrows - 1) * res_stride + hidden) * 2);
      rrs = make_rsrc(res_rows + row0 * res_stride, rbytes);
      roff = (uint32_t)rib * (uint32_t)res_stride * 2u + lofs;
    }

    // TAIL: the lane's edge vector (head or tail); the e*off offsets address
    // the edge vector in each stream, kOOB elsewhere
    uint32_t exoff = kOOB, eroff = kOOB, ewoff = kOOB, eb = 0, eq = 0;
    int elo = 0, ehi = 0;
    bool eok = false;
    if constexpr (TAIL) {
      const uint32_t xrow = xoff - lofs, rrow = roff - lofs;
#pragma unroll
      for (int k = 0; k < VPL; ++k) vec_ok[k] = (k * LPR + lane) < nb;
      xoff += wshift;
      if constexpr (RES) roff += wshift;
      // the head goes to the lane holding body vector 0 (slot rp), the tail
      // to the lane holding body vector nb - 1 (slot rp - 1, or nb - 1
      // unrotated), or to the next lane when that is the head's
      const int hl = rp;
      int tl = rp > 0 ? rp - 1 : (nb - 1) & (LPR - 1);
      if (delta > 0 && tl == hl) tl = hl + 1;
      if (delta > 0 && lane == hl) {
        eok = row_ok; elo = 0; ehi = 8 - delta;
      } else if (t > 0 && lane == tl) {
        eok = row_ok; elo = 8 - t; ehi = 8;
        eb = 2u * (uint32_t)hidden - 16u;
        eq = (uint32_t)hidden - 8u;
      }
      if (eok) {
        exoff = xrow + eb;
        if constexpr (RES) eroff = rrow + eb;
        ewoff = eb;
      }
    }

    // WLDS: the first row group loads the whole weight (aligned) before its
    // row loads and writes it to LDS after them; the values stay live only
    // within this iteration
    u32x4 wst[NST], wtl = {};
    if constexpr (WLDS) {
      if (!staged) {
#pragma unroll
        for (int i = 0; i < NST; ++i) {
          const int v = tid + i * BLOCK;
          wst[i] = load16<0>(wrs, v < nvec ? (uint32_t)v * 16u : kOOB);
        }
        // the elements past the last whole vector, from the weight's last 16 bytes
        if ((hidden & 7) != 0 && tid == BLOCK - 1) wtl = load16<0>(wrs, 2u * (uint32_t)hidden - 16u);
      }
    }
    u32x4 xv[VPL], rv[VPL], wv[VPL];
    if constexpr (ALTW || ALTG) {
      if (ALTW ? (wave & 1) != 0 : (blockIdx.x & 1) != 0) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) rv[k] = load16<RLAUX>(rrs, (row_ok && vec_ok[k]) ? roff + vk(k) : kOOB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < VPL; ++k) xv[k] = load16<XLAUX>(xrs, (row_ok && vec_ok[k]) ? xoff + vk(k) : kOOB);
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int k = 0; k < VPL; ++k) xv[k] = load16<XLAUX>(xrs, (row_ok && vec_ok[k]) ? xoff + vk(k) : kOOB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < VPL; ++k) rv[k] = load16<RLAUX>(rrs, (row_ok && vec_ok[k]) ? roff + vk(k) : kOOB);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (RFIRST) {
      // all of the residual's vectors, then all of the input's (the
      // scheduling barriers keep the two groups apart)
#pragma unroll
      for (int k = 0; k < VPL; ++k) rv[k] = load16<RLAUX>(rrs, (row_ok && vec_ok[k]) ? roff + vk(k) : kOOB);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < VPL; ++k) xv[k] = load16<XLAUX>(xrs, (row_ok && vec_ok[k]) ? xoff + vk(k) : kOOB);
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const bool ok = row_ok && vec_ok[k];
        xv[k] = load16<XLAUX>(xrs, ok ? xoff + vk(k) : kOOB);
        if constexpr (RES) rv[k] = load16<RLAUX>(rrs, ok ? roff + vk(k) : kOOB);
      }
    }
    // TAIL: the edge vector's loads, by the lanes that hold one only (a
    // branch, so that the other waves issue none: measured up to 12% faster
    // than loads at out-of-range offsets from every lane, at 16K-17K)
    u32x4 txv = {}, trv = {}, twv = {};
    if constexpr (TAIL) {
      if (eok) {
        txv = load16<XLAUX>(xrs, exoff);
        if constexpr (RES) trv = load16<RLAUX>(rrs, eroff);
      }
    }
    if constexpr (!WLATE) {
#pragma unroll
      for (int k = 0; k < VPL; ++k)
        wv[k] = load16<0>(wrs, (TAIL && !vec_ok[k]) ? kOOB : lofs + vk(k) + wshift);
      if constexpr (TAIL) {
        if (eok) twv = load16<0>(wrs, ewoff);
      }
    }
    if constexpr (WLDS) {
      // (the row-sum barrier below makes these writes visible to the workgroup)
      if (!staged) {
#pragma unroll
        for (int i = 0; i < NST; ++i) {
          const int v = tid + i * BLOCK;
          if (v < nvec) wlds[v] = wst[i];
        }
        if ((hidden & 7) != 0 && tid == BLOCK - 1) {
          uint16_t* const w16 = reinterpret_cast<uint16_t*>(wlds);
          const int r = hidden & 7;
#pragma unroll
          for (int i = 0; i < 7; ++i) {
            if (i < r) {
              const int e = i + 8 - r;  // element 8 * nvec + i among the last 8
              w16[8 * nvec + i] = (uint16_t)(wtl[e >> 1] >> ((e & 1) * 16));
            }
          }
        }
        staged = true;
      }
    }

    // The written streams' resources, after the row loads have been issued:
    // the arguments of modes 2-6 come from FusedArgs (not preloaded), read
    // here through opaque() so that neither they nor what is computed from
    // them moves ahead of the loads, which then wait for no scalar load.
    // Modes 0 and 1 write through preloaded arguments and take no barrier
    // (with it the compiler kept 64 x 8's unpacked rows live, 120 -> 189
    // VGPRs), nor does the LDS tier, whose weight loads then trail the row
    // loads (1-1.6% slower at 16K-32K, two builds side by side).
    // srs/soff: residual stores; ors/ooff: output; xsrs/xsoff: block scales (MX, MODE 7)
    if constexpr (MODE >= 2 && LDSV == 0) __builtin_amdgcn_sched_barrier(0);
    __amdgpu_buffer_rsrc_t srs = rrs, ors = xrs, xsrs = xrs;
    uint32_t soff = roff, ooff = xoff, xsoff = 0, esoff = eroff, eooff = exoff;
    uint32_t gs = 4;  // MODE 7: bytes between a row's consecutive scales
    // MODE 2: the caller's upper bound on the row maximum, or the one given
    // scale, loaded while the row loads are in flight rather than when the
    // output phase needs it (no bound: NaN, which bounds nothing)
    float ubound = __builtin_nanf("");
    float given_scale = 0.0f;
    bool has_given = false;
    if constexpr (MODE == 2) {
      const float* const ub = opaque(a.scale_ub);
      if (ub != nullptr) ubound = *ub;
      const float* const given = opaque(a.static_scale);
      has_given = given != nullptr;
      if (has_given) given_scale = *given;
    }
    if constexpr (MODE == 3) {
      uint16_t* const ro = opaque(a.res_out);
      const int64_t rs = opaque(a.res_out_stride);
      const uint32_t sbytes = (uint32_t)(((int64_t)(nrows - 1) * rs + hidden) * 2);
      srs = make_rsrc(ro + row0 * rs, sbytes);
      const uint32_t srow = (uint32_t)rib * (uint32_t)rs * 2u;
      soff = srow + lofs + wshift;
      esoff = eok ? srow + eb : kOOB;
    }
    if constexpr (MODE == 2 || BLOCKQ) {
      constexpr uint32_t QB = MODE == 6 ? 4u : 8u;  // output bytes per 8-element vector
      uint8_t* const qp = opaque(a.q);
      const int64_t qs = opaque(a.q_stride);
      const uint32_t qbytes = (uint32_t)((int64_t)(nrows - 1) * qs + hidden * (int64_t)QB / 8);
      ors = make_rsrc(qp + row0 * qs, qbytes);
      const uint32_t qrow = (uint32_t)rib * (uint32_t)qs;
      ooff = qrow + (uint32_t)(lane - rp) * QB + (TAIL ? (uint32_t)(8 * j0 - delta) : 0u);
      eooff = eok ? qrow + eq : kOOB;
    }
    if constexpr (MX) {
      uint8_t* const sp = opaque(a.mx_scale);
      const int64_t ss = opaque(a.mx_scale_stride);
      const uint32_t sbytes = (uint32_t)((int64_t)(nrows - 1) * ss + hidden / 32);
      xsrs = make_rsrc(sp + row0 * ss, sbytes);
      // one lane of each quad writes its block's scale byte
      xsoff = (lane & 3) == 0 ? (uint32_t)rib * (uint32_t)ss + (uint32_t)lane / 4u : kOOB;
    }
    if constexpr (GQ) {
      // float32 scales, one per 128 elements; scale (row, group) at byte
      // row * mx_scale_stride + group * mx_group_stride (row-major scales:
      // group stride 4; column-major: row stride 4)
      uint8_t* const sp = opaque(a.mx_scale);
      const int64_t ss = opaque(a.mx_scale_stride);
      gs = (uint32_t)opaque(a.mx_group_stride);
      const uint32_t sbytes = (uint32_t)((int64_t)(nrows - 1) * ss + (int64_t)(hidden / 128 - 1) * gs + 4);
      xsrs = make_rsrc(sp + row0 * ss, sbytes);
      // the first lane of each 16 writes its group's scale
      xsoff = (lane & 15) == 0 ? (uint32_t)rib * (uint32_t)ss + (uint32_t)(lane / 16) * gs : kOOB;
    }
    if constexpr (MODE == 1) {
      // no residual: its (preloaded) arguments carry the output rows
      const uint32_t obytes = (uint32_t)(((int64_t)(nrows - 1) * res_stride + hidden) * 2);
      ors = make_rsrc(res_rows + row0 * res_stride, obytes);
      const uint32_t orow = (uint32_t)rib * (uint32_t)res_stride * 2u;
      ooff = orow + lofs + wshift;
      eooff = eok ? orow + eb : kOOB;
    } else if constexpr (OUT16) {
      uint16_t* const op = opaque(a.out);
      const int64_t os = opaque(a.out_stride);
      const uint32_t obytes = (uint32_t)(((int64_t)(nrows - 1) * os + hidden) * 2);
      ors = make_rsrc(op + row0 * os, obytes);
      const uint32_t orow = (uint32_t)rib * (uint32_t)os * 2u;
      ooff = orow + lofs + wshift;
      eooff = eok ? orow + eb : kOOB;
    }

    if constexpr (MODE == 4) {
      // x := rne(sum of the parts), accumulated in fp32 in part order and
      // rounded once, for groups of at most 2 vector slots at a time when a
      // lane holds more than 4 (8 slots would need 64 fp32 accumulators per
      // lane: past the VGPR budget of the wide shapes); the tail goes with the
      // last group.  The unrolled loops keep every parts[] and slot index a
      // constant.
      // FLAGS bit 15 (the latency rows, few rows per call): each group's loads
      // of every part are issued before the first part is added, so the parts
      // cost one memory round trip rather than one each (G <= 2: at most 7 x 2
      // vectors in flight per lane)
      constexpr bool PF = (FLAGS & 32768) != 0;
      constexpr int G = PF ? (VPL < 2 ? VPL : 2) : (VPL <= 4 ? VPL : 2);
#pragma unroll
      for (int k0 = 0; k0 < VPL; k0 += G) {
        const bool with_tail = TAIL && k0 + G >= VPL;
        float acc[G][8], tacc[8];
#pragma unroll
        for (int i = 0; i < G; ++i) {
          const int k = k0 + i < VPL ? k0 + i : 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][2 * j] = F::lo(xv[k][j]);
            acc[i][2 * j + 1] = F::hi(xv[k][j]);
          }
        }
        if (with_tail) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            tacc[2 * j] = F::lo(txv[j]);
            tacc[2 * j + 1] = F::hi(txv[j]);
          }
        }
        if constexpr (PF) {
          const int np = opaque(a.nparts);
          u32x4 ppv[HPRMS_MAX_PARTS - 1][G], ptv[HPRMS_MAX_PARTS - 1];
#pragma unroll
          for (int g = 1; g < HPRMS_MAX_PARTS; ++g) {
            if (g < np) {
              const __amdgpu_buffer_rsrc_t prs = make_rsrc(opaque(a.parts[g]) + row0 * x_stride, xbytes);
#pragma unroll
              for (int i = 0; i < G; ++i) {
                const int k = k0 + i < VPL ? k0 + i : 0;
                ppv[g - 1][i] = load16<LAUX>(prs, (k0 + i < VPL && row_ok && vec_ok[k]) ? xoff + vk(k) : kOOB);
              }
              ptv[g - 1] = u32x4{};
              if (with_tail && eok) ptv[g - 1] = load16<LAUX>(prs, exoff);
            }
          }
          // added in part order, as below
#pragma unroll
          for (int g = 1; g < HPRMS_MAX_PARTS; ++g) {
            if (g < np) {
#pragma unroll
              for (int i = 0; i < G; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  acc[i][2 * j] += F::lo(ppv[g - 1][i][j]);
                  acc[i][2 * j + 1] += F::hi(ppv[g - 1][i][j]);
                }
              if (with_tail) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  tacc[2 * j] += F::lo(ptv[g - 1][j]);
                  tacc[2 * j + 1] += F::hi(ptv[g - 1][j]);
                }
              }
            }
          }
        }
#pragma unroll
        for (int g = 1; g < HPRMS_MAX_PARTS; ++g) {
          if (PF) break;
          if (g >= opaque(a.nparts)) break;
          const __amdgpu_buffer_rsrc_t prs = make_rsrc(opaque(a.parts[g]) + row0 * x_stride, xbytes);
          u32x4 pv[G], tpv = {};
#pragma unroll
          for (int i = 0; i < G; ++i) {
            const int k = k0 + i < VPL ? k0 + i : 0;
            pv[i] = load16<LAUX>(prs, (k0 + i < VPL && row_ok && vec_ok[k]) ? xoff + vk(k) : kOOB);
          }
          if (with_tail && eok) tpv = load16<LAUX>(prs, exoff);
#pragma unroll
          for (int i = 0; i < G; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc[i][2 * j] += F::lo(pv[i][j]);
              acc[i][2 * j + 1] += F::hi(pv[i][j]);
            }
          if (with_tail) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              tacc[2 * j] += F::lo(tpv[j]);
              tacc[2 * j + 1] += F::hi(tpv[j]);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
          if (k0 + i < VPL) {
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[k0 + i < VPL ? k0 + i : 0][j] = F::pack(acc[i][2 * j], acc[i][2 * j + 1]);
          }
        }
        if (with_tail) {
#pragma unroll
          for (int j = 0; j < 4; ++j) txv[j] = F::pack(tacc[2 * j], tacc[2 * j + 1]);
        }
      }
    }

    float ss0 = 0.0f, ss1 = 0.0f;
    u32x4 sv[VREG > 0 ? VREG : 1];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      u32x4 s;
      if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t p = F::pack(F::lo(xv[k][j]) + F::lo(rv[k][j]), F::hi(xv[k][j]) + F::hi(rv[k][j]));
          s[j] = p;
          const float b0 = F::lo(p), b1 = F::hi(p);
          ss0 = __builtin_fmaf(b0, b0, ss0);
          ss1 = __builtin_fmaf(b1, b1, ss1);
        }
        const bool ok = row_ok && vec_ok[k];
        store16<RSAUX>(s, srs, ok ? soff + vk(k) : kOOB);
      } else {
        s = xv[k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float b0 = F::lo(s[j]), b1 = F::hi(s[j]);
          ss0 = __builtin_fmaf(b0, b0, ss0);
          ss1 = __builtin_fmaf(b1, b1, ss1);
        }
      }
      if (k < VREG) sv[k < VREG ? k : 0] = s;
      else spill[(k - VREG) * BLOCK + tid] = s;
    }
    u32x4 tsv = {};
    if constexpr (TAIL) {
      // only the edge vector's elements elo <= e < ehi are not held by a body
      // vector (a select, so that a masked infinity adds 0 and not NaN)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t p = RES ? F::pack(F::lo(txv[j]) + F::lo(trv[j]), F::hi(txv[j]) + F::hi(trv[j])) : txv[j];
        tsv[j] = p;
        const float b0 = (2 * j >= elo && 2 * j < ehi) ? F::lo(p) : 0.0f;
        const float b1 = (2 * j + 1 >= elo && 2 * j + 1 < ehi) ? F::hi(p) : 0.0f;
        ss0 = __builtin_fmaf(b0, b0, ss0);
        ss1 = __builtin_fmaf(b1, b1, ss1);
      }
      if constexpr (RES) store16<RSAUX>(tsv, srs, esoff);
    }

    if constexpr (WLATE) {
      if constexpr (!WLDS) {
#pragma unroll
        for (int k = 0; k < VPL; ++k)
          wv[k] = load16<0>(wrs, (TAIL && !vec_ok[k]) ? kOOB : lofs + vk(k) + wshift);
      }
      if constexpr (TAIL) {
        if (eok) twv = load16<0>(wrs, ewoff);
      }
    }

    float tot = group_sum<GW>(ss0 + ss1);
    if constexpr (WPR > 1) {
      if ((tid & 63) == 0) red[buf][wave] = tot;
      __syncthreads();
      const int w0 = (wave / WPR) * WPR;
      tot = red[buf][w0];
#pragma unroll
      for (int j = 1; j < WPR; ++j) tot += red[buf][w0 + j];
      buf ^= 1;
    }
    if constexpr (WLDS) {
      // slot k's vector starts at byte lofs + vk(k) + wshift of the weight:
      // the five dwords from the one holding its first element, shifted by
      // 0 or 16 bits (wshift is even; the same phase for every slot)
      const uint32_t* const wd = reinterpret_cast<const uint32_t*>(wlds);
      const uint32_t sh = (wshift & 3u) * 8u;
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const uint32_t i = vec_ok[k] ? (lofs + vk(k) + wshift) >> 2 : 0u;
        uint32_t d[5];
#pragma unroll
        for (int j = 0; j < 5; ++j) d[j] = wd[i + j];
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[k][j] = __builtin_amdgcn_alignbit(d[j + 1], d[j], sh);
      }
    }
    const float inv = 1.0f / __builtin_sqrtf(tot / hidden_f + eps);
    // FLAGS bit 19 (bench library): the output phase at raised wave priority
    if constexpr ((FLAGS & 524288) != 0) __builtin_amdgcn_s_setprio(3);

    if constexpr (MX) {
      constexpr int EMAX = MODE == 5 ? 8 : 2;
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const u32x4 s = k < VREG ? sv[k < VREG ? k : 0] : spill[(k - VREG) * BLOCK + tid];
        u32x4 y;
        uint32_t m2 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y[j] = F::pack((olo(s[j]) * inv) * F::lo(wv[k][j]), (ohi(s[j]) * inv) * F::hi(wv[k][j]));
          const uint32_t mag = y[j] & 0x7fff7fffu;
          m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(mag & 0xffffu, mag >> 16));
        }
        // the block maximum as binary32: its exponent field is floor(log2) + 127
        // (0 for zero and for bf16 subnormals, which clamp; 255 for NaN / inf)
        const uint32_t e32 = __float_as_uint(F::one((uint16_t)quad_max_u32(m2))) >> 23;
        int sexp = (int)e32 - 127 - EMAX;
        if (e32 == 0 || sexp < -127) sexp = -127;
        const bool bad = e32 == 255u;
        const float mul = bad ? 1.0f : __uint_as_float((uint32_t)(127 - sexp) << 23);
        const bool ok = row_ok && vec_ok[k];
        // a wave writes 16 consecutive scale bytes: default cache policy, so
        // that L2 merges the pieces of a line before it goes to memory
        store1<0>((uint8_t)(bad ? 0xFFu : (uint32_t)(sexp + 127)), xsrs,
                  ok && xsoff != kOOB ? xsoff + (uint32_t)(k * (LPR / 4)) : kOOB);
        if constexpr (MODE == 5) {
          u32x2 q;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t y0 = y[2 * h], y1 = y[2 * h + 1];
            q[h] = pack_e4m3x4(clamp_e4m3(F::lo(y0) * mul), clamp_e4m3(F::hi(y0) * mul),
                               clamp_e4m3(F::lo(y1) * mul), clamp_e4m3(F::hi(y1) * mul));
          }
          store8<OSAUX>(q, ors, ok ? ooff + k * (LPR * 8u) : kOOB);
        } else {
          uint32_t q = 0;
          q = cvt_e2m1x2<0>(q, F::lo(y[0]) * mul, F::hi(y[0]) * mul);
          q = cvt_e2m1x2<1>(q, F::lo(y[1]) * mul, F::hi(y[1]) * mul);
          q = cvt_e2m1x2<2>(q, F::lo(y[2]) * mul, F::hi(y[2]) * mul);
          q = cvt_e2m1x2<3>(q, F::lo(y[3]) * mul, F::hi(y[3]) * mul);
          store4<OSAUX>(q, ors, ok ? ooff + k * (LPR * 4u) : kOOB);
        }
      }
    } else if constexpr (GQ) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const u32x4 s = k < VREG ? sv[k < VREG ? k : 0] : spill[(k - VREG) * BLOCK + tid];
        u32x4 y;
        uint32_t m2 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y[j] = F::pack((olo(s[j]) * inv) * F::lo(wv[k][j]), (ohi(s[j]) * inv) * F::hi(wv[k][j]));
          const uint32_t mag = y[j] & 0x7fff7fffu;
          m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(mag & 0xffffu, mag >> 16));
        }
        // the group's maximum magnitude: the 16 lanes of a DPP row hold its
        // 16 vectors (sign-magnitude patterns order like their values, NaN
        // above inf)
        const float amax = F::one((uint16_t)group_max_u32<16>(m2));
        float sc = amax / 448.0f;
        if (sc < 1.17549435e-38f) sc = 1.17549435e-38f;  // FLT_MIN; NaN stays NaN
        const float isc = 1.0f / sc;
        const bool ok = row_ok && vec_ok[k];
        // default cache policy, so that L2 merges a row's scales into lines
        store4<0>(__float_as_uint(sc), xsrs, ok && xsoff != kOOB ? xsoff + (uint32_t)(k * (LPR / 16)) * gs : kOOB);
        u32x2 q;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t y0 = y[2 * h], y1 = y[2 * h + 1];
          q[h] = pack_e4m3x4(clamp_e4m3(F::lo(y0) * isc), clamp_e4m3(F::hi(y0) * isc),
                             clamp_e4m3(F::lo(y1) * isc), clamp_e4m3(F::hi(y1) * isc));
        }
        store8<OSAUX>(q, ors, ok ? ooff + k * (LPR * 8u) : kOOB);
      }
    } else if constexpr (MODE != 2) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const u32x4 s = k < VREG ? sv[k < VREG ? k : 0] : spill[(k - VREG) * BLOCK + tid];
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = F::pack((olo(s[j]) * inv) * F::lo(wv[k][j]), (ohi(s[j]) * inv) * F::hi(wv[k][j]));
        const bool ok = row_ok && vec_ok[k];
        store16<OSAUX>(o, ors, ok ? ooff + vk(k) : kOOB);
      }
      if constexpr (TAIL) {
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = F::pack((olo(tsv[j]) * inv) * F::lo(twv[j]), (ohi(tsv[j]) * inv) * F::hi(twv[j]));
        store16<OSAUX>(o, ors, eooff);
      }
    } else {
      // y in 16-bit form, kept in the registers x came in; the row maximum of
      // |y| over the valid vectors, as packed 16-bit magnitudes
      uint32_t m2 = 0;
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const u32x4 s = k < VREG ? sv[k < VREG ? k : 0] : spill[(k - VREG) * BLOCK + tid];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xv[k][j] = F::pack((olo(s[j]) * inv) * F::lo(wv[k][j]), (ohi(s[j]) * inv) * F::hi(wv[k][j]));
        if (row_ok && vec_ok[k]) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t mag = xv[k][j] & 0x7fff7fffu;
            const uint32_t lo = mag & 0xffffu, hi = mag >> 16;
            m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(lo, hi));
          }
        }
      }
      if constexpr (TAIL) {
        // the edge vector's elements outside [elo, ehi) repeat ones already
        // counted: harmless for a maximum
#pragma unroll
        for (int j = 0; j < 4; ++j)
          txv[j] = F::pack((olo(tsv[j]) * inv) * F::lo(twv[j]), (ohi(tsv[j]) * inv) * F::hi(twv[j]));
        if (eok) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t mag = txv[j] & 0x7fff7fffu;
            m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(mag & 0xffffu, mag >> 16));
          }
        }
      }
      float isc;
      if (has_given) {
        // one scale for every row, given by the caller: no row maximum (the
        // branch is uniform over the workgroup, so no barrier is skipped by
        // part of it)
        isc = 1.0f / given_scale;
      } else {
        uint32_t mx = group_max_u32<GW>(m2);
        if constexpr (WPR > 1) {
          if ((tid & 63) == 0) red[buf][wave] = __builtin_bit_cast(float, mx);
          __syncthreads();
          const int w0 = (wave / WPR) * WPR;
#pragma unroll
          for (int j = 0; j < WPR; ++j)
            mx = __builtin_elementwise_max(mx, __builtin_bit_cast(uint32_t, red[buf][w0 + j]));
          buf ^= 1;
        }
        float amax = F::one((uint16_t)mx);
        if (amax > ubound) amax = ubound;  // the caller's bound (a NaN maximum stays NaN)
        float sc = amax / 448.0f;
        if (sc < 1.17549435e-38f) sc = 1.17549435e-38f;  // FLT_MIN; NaN stays NaN
        isc = 1.0f / sc;
        if (row_ok && lane == 0) opaque(a.scale)[row0 + rib] = sc;
      }
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        u32x2 q;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t y0 = xv[k][2 * h], y1 = xv[k][2 * h + 1];
          q[h] = pack_e4m3x4(clamp_e4m3(F::lo(y0) * isc), clamp_e4m3(F::hi(y0) * isc),
                             clamp_e4m3(F::lo(y1) * isc), clamp_e4m3(F::hi(y1) * isc));
        }
        const bool ok = row_ok && vec_ok[k];
        store8<OSAUX>(q, ors, ok ? ooff + k * (LPR * 8u) + (k == 0 ? wrap * 8u : 0u) : kOOB);
      }
      if constexpr (TAIL) {
        u32x2 q;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t y0 = txv[2 * h], y1 = txv[2 * h + 1];
          q[h] = pack_e4m3x4(clamp_e4m3(F::lo(y0) * isc), clamp_e4m3(F::hi(y0) * isc),
                             clamp_e4m3(F::lo(y1) * isc), clamp_e4m3(F::hi(y1) * isc));
        }
        store8<OSAUX>(q, ors, eooff);
      }
    }
    if constexpr ((FLAGS & 524288) != 0) __builtin_amdgcn_s_setprio(0);
    g += grid;
    if (g >= ngroups) break;
  }
  if constexpr (TIMELINE) {
    __builtin_amdgcn_s_waitcnt(0);  // every load and store of this wave has completed
    __syncthreads();
    if (tid == 0) {
      int64_t* t = a.timeline + 4 * (int64_t)blockIdx.x;
      t[0] = (int64_t)t_start;
      t[1] = (int64_t)__builtin_amdgcn_s_memrealtime();
      t[2] = (int64_t)(uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID: wave, SIMD, CU, SH, SE
      t[3] = (int64_t)(uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 20);  // XCC_ID
    }
  }
}

// General kernel: any hidden, any alignment, any row strides.  One workgroup
// per row (grid-stride), element-wise 2-byte accesses; the second pass
// re-reads the residual row this same thread has just written (program order
// makes its own store visible), so nothing limits hidden.
struct GeneralArgs {
  const uint16_t* x;
  uint16_t* out;
  uint16_t* res;
  const uint16_t* w;
  int64_t rows;
  int64_t x_stride;
  int64_t out_stride;
  int64_t res_stride;
  int64_t hidden;
  float hidden_f;
  float eps;
  uint8_t* q;        // MODE 2
  float* scale;      // MODE 2
  const float* static_scale;  // MODE 2: as FusedArgs::static_scale
  const float* scale_ub;      // MODE 2: as FusedArgs::scale_ub
  int64_t q_stride;  // MODE 2
  uint16_t* res_out;  // MODE 3
  int64_t res_out_stride;
  int32_t nparts;    // MODE 4
  const uint16_t* parts[HPRMS_MAX_PARTS];
};

template <int DT, int MODE>
__global__ __launch_bounds__(256) void fused_general_kernel(GeneralArgs a) {
  using F = Fmt<DT>;
  __shared__ float red[2][4];
  const int tid = threadIdx.x;
  int buf = 0;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* x = a.x + row * a.x_stride;
    uint16_t* o = a.out + row * a.out_stride;
    const uint16_t* r = MODE != 1 ? a.res + row * a.res_stride : nullptr;
    // where the rounded sum goes (and is read back from by the output pass)
    uint16_t* rs = MODE == 3 ? a.res_out + row * a.res_out_stride
                   : MODE != 1 ? a.res + row * a.res_stride : nullptr;
    float ss = 0.0f;
    for (int64_t j = tid; j < a.hidden; j += 256) {
      float v;
      if constexpr (MODE != 1) {
        float xj = F::one(x[j]);
        if constexpr (MODE == 4) {
#pragma unroll
          for (int g = 1; g < HPRMS_MAX_PARTS; ++g) {
            if (g >= a.nparts) break;
            xj += F::one(a.parts[g][row * a.x_stride + j]);
          }
          xj = F::one(F::pack1(xj));
        }
        const uint16_t s = F::pack1(xj + F::one(r[j]));
        rs[j] = s;
        v = F::one(s);
      } else {
        v = F::one(x[j]);
      }
      ss = __builtin_fmaf(v, v, ss);
    }
    float tot = group_sum<64>(ss);
    if ((tid & 63) == 0) red[buf][tid >> 6] = tot;
    __syncthreads();
    tot = ((red[buf][0] + red[buf][1]) + red[buf][2]) + red[buf][3];
    buf ^= 1;
    const float inv = 1.0f / __builtin_sqrtf(tot / a.hidden_f + a.eps);
    if constexpr (MODE != 2) {
      for (int64_t j = tid; j < a.hidden; j += 256) {
        const float v = MODE == 1 ? F::one(x[j]) : F::one(rs[j]);
        o[j] = F::pack1((v * inv) * F::one(a.w[j]));
      }
    } else {
      // y is recomputed in each pass from the residual this thread wrote, so
      // both passes see the same bits
      float isc;
      if (a.static_scale != nullptr) {
        isc = 1.0f / *a.static_scale;   // one given scale for every row (uniform branch)
      } else {
        uint32_t m = 0;
        for (int64_t j = tid; j < a.hidden; j += 256)
          m = __builtin_elementwise_max(m, (uint32_t)(F::pack1((F::one(rs[j]) * inv) * F::one(a.w[j])) & 0x7fffu));
        uint32_t mx = group_max_u32<64>(m);
        if ((tid & 63) == 0) red[buf][tid >> 6] = __builtin_bit_cast(float, mx);
        __syncthreads();
        for (int j = 0; j < 4; ++j) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(uint32_t, red[buf][j]));
        buf ^= 1;
        float amax = F::one((uint16_t)mx);
        if (a.scale_ub != nullptr && amax > *a.scale_ub) amax = *a.scale_ub;  // the caller's upper bound
        float sc = amax / 448.0f;
        if (sc < 1.17549435e-38f) sc = 1.17549435e-38f;  // FLT_MIN; NaN stays NaN
        isc = 1.0f / sc;
        if (tid == 0) a.scale[row] = sc;
      }
      uint8_t* qr = a.q + row * a.q_stride;
      for (int64_t j = tid; j < a.hidden; j += 256) {
        const float y = F::one(F::pack1((F::one(rs[j]) * inv) * F::one(a.w[j])));
        qr[j] = (uint8_t)(pack_e4m3x4(clamp_e4m3(y * isc), 0.0f, 0.0f, 0.0f) & 0xffu);
      }
    }
  }
}

// General kernel, register-resident form: any alignment and row strides,
// hidden <= BLOCK * E (the host picks E so that at most one element slot per
// thread lies wholly past the row).  One workgroup per row (grid-stride);
// thread t owns elements t, t + BLOCK, ..., t + (E-1) * BLOCK (each wave
// instruction moves 128 contiguous bytes), issues all its loads first and
// keeps the row in registers, so the row is read once and written once, as in
// the vector tiers.  Accesses are 2-byte buffer loads and stores through
// resources sized to the row: elements past its end read as 0 and their
// stores are dropped by the hardware range check, so the code is straight-line
// (a branch per slot would make the wait counters conservative and serialise
// the stores).  Same modes 0-4 and arithmetic as fused_general_kernel.
template <int DT, int MODE, int BLOCK, int E>
__global__ __launch_bounds__(BLOCK) void fused_general_reg_kernel(GeneralArgs a) {
  static_assert(MODE >= 0 && MODE <= 4 && BLOCK % 64 == 0, "mode / block");
  using F = Fmt<DT>;
  constexpr int NW = BLOCK / 64;
  __shared__ float red[2][NW];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const uint32_t rowbytes = (uint32_t)a.hidden * 2u;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, rowbytes);
  int buf = 0;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x + row * a.x_stride, rowbytes);
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(a.out + row * a.out_stride, rowbytes);
    __amdgpu_buffer_rsrc_t rrs = xrs, srs = xrs;
    if constexpr (MODE != 1) {
      rrs = make_rsrc(a.res + row * a.res_stride, rowbytes);
      srs = MODE == 3 ? make_rsrc(a.res_out + row * a.res_out_stride, rowbytes) : rrs;
    }
    // one 32-bit register per element: 16-bit arrays would be packed in
    // pairs, and the packing waits for each load
    uint32_t xv[E], rv[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const uint32_t off = (uint32_t)(tid + k * BLOCK) * 2u;
      xv[k] = __builtin_amdgcn_raw_buffer_load_b16(xrs, off, 0, 0);
      if constexpr (MODE != 1) rv[k] = __builtin_amdgcn_raw_buffer_load_b16(rrs, off, 0, 0);
    }
    float acc[MODE == 4 ? E : 1];
    if constexpr (MODE == 4) {
#pragma unroll
      for (int k = 0; k < E; ++k) acc[k] = F::one((uint16_t)xv[k]);
#pragma unroll
      for (int g = 1; g < HPRMS_MAX_PARTS; ++g) {
        if (g >= a.nparts) break;
        const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.parts[g] + row * a.x_stride, rowbytes);
#pragma unroll
        for (int k = 0; k < E; ++k)
          acc[k] += F::one(__builtin_amdgcn_raw_buffer_load_b16(prs, (uint32_t)(tid + k * BLOCK) * 2u, 0, 0));
      }
    }
    float sv[E];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if constexpr (MODE != 1) {
        const float xj = MODE == 4 ? F::one(F::pack1(acc[MODE == 4 ? k : 0])) : F::one((uint16_t)xv[k]);
        const uint16_t s = F::pack1(xj + F::one((uint16_t)rv[k]));
        __builtin_amdgcn_raw_buffer_store_b16(s, srs, (uint32_t)(tid + k * BLOCK) * 2u, 0, 0);
        sv[k] = F::one(s);
      } else {
        sv[k] = F::one((uint16_t)xv[k]);
      }
      ss = __builtin_fmaf(sv[k], sv[k], ss);   // elements past the row are 0
    }
    float tot = group_sum<64>(ss);
    if ((tid & 63) == 0) red[buf][wave] = tot;
    __syncthreads();
    tot = red[buf][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) tot += red[buf][w];
    const float inv = 1.0f / __builtin_sqrtf(tot / a.hidden_f + a.eps);
    // every weight load before the first output store: a load after a store
    // could not be moved above it (the compiler cannot rule out aliasing)
#pragma unroll
    for (int k = 0; k < E; ++k) rv[k] = __builtin_amdgcn_raw_buffer_load_b16(wrs, (uint32_t)(tid + k * BLOCK) * 2u, 0, 0);
    if constexpr (MODE != 2) {
#pragma unroll
      for (int k = 0; k < E; ++k)
        __builtin_amdgcn_raw_buffer_store_b16(F::pack1((sv[k] * inv) * F::one((uint16_t)rv[k])), ors,
                                              (uint32_t)(tid + k * BLOCK) * 2u, 0, 0);
    } else {
      uint32_t m = 0;
#pragma unroll
      for (int k = 0; k < E; ++k) {
        xv[k] = F::pack1((sv[k] * inv) * F::one((uint16_t)rv[k]));  // the 16-bit output (0 past the row)
        m = __builtin_elementwise_max(m, xv[k] & 0x7fffu);
      }
      float isc;
      if (a.static_scale != nullptr) {
        isc = 1.0f / *a.static_scale;   // one given scale for every row (uniform branch)
      } else {
        uint32_t mx = group_max_u32<64>(m);
        buf ^= 1;
        if ((tid & 63) == 0) red[buf][wave] = __builtin_bit_cast(float, mx);
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(uint32_t, red[buf][w]));
        float amax = F::one((uint16_t)mx);
        if (a.scale_ub != nullptr && amax > *a.scale_ub) amax = *a.scale_ub;  // the caller's upper bound
        float sc = amax / 448.0f;
        if (sc < 1.17549435e-38f) sc = 1.17549435e-38f;  // FLT_MIN; NaN stays NaN
        isc = 1.0f / sc;
        if (tid == 0) a.scale[row] = sc;
      }
      const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q + row * a.q_stride, (uint32_t)a.hidden);
#pragma unroll
      for (int k = 0; k < E; ++k)
        __builtin_amdgcn_raw_buffer_store_b8(
            (uint8_t)(pack_e4m3x4(clamp_e4m3(F::one((uint16_t)xv[k]) * isc), 0.0f, 0.0f, 0.0f) & 0xffu), qrs,
            (uint32_t)(tid + k * BLOCK), 0, 0);
    }
    buf ^= 1;
  }
}

// Launches the general tier for `dtype` (HPRMS_DTYPE_*) and mode 0-4 on
// `stream`: the register-resident kernel up to hidden = 16384, the two-pass
// kernel above (hprms_general.hip).  Launch errors are left for the caller.
void launch_general_kernels(const GeneralArgs& a, int dtype, int mode, int64_t grid, hipStream_t stream);

// ---- streamer ------------------------------------------------------------------
struct StreamArgs {
  uint16_t* out;
  const uint16_t* in;
  int64_t rows;
  int64_t hidden;
  int64_t out_stride;
  int64_t in_stride;
  int64_t nvec;  // flat kernel: total 16-byte vectors; row kernel: vectors per row
};

template <int DT, int OP>
__device__ __forceinline__ uint32_t stream_op2(uint32_t w) {
  if constexpr (OP == HPRMS_STREAM_COPY) {
    return w;
  } else {
    // ReLU on two 16-bit lanes: strictly negative (sign set, magnitude in
    // (0, inf]) becomes +0; -0 and NaN pass through.
    constexpr uint32_t inf = DT == HPRMS_DTYPE_BF16 ? 0x7f80u : 0x7c00u;
    const uint32_t m0 = w & 0x7fffu, m1 = (w >> 16) & 0x7fffu;
    const bool z0 = (w & 0x8000u) && m0 != 0 && m0 <= inf;
    const bool z1 = (w & 0x80000000u) && m1 != 0 && m1 <= inf;
    return (z0 ? 0u : (w & 0xffffu)) | (z1 ? 0u : (w & 0xffff0000u));
  }
}

template <int DT, int OP>
__device__ __forceinline__ uint16_t stream_op1(uint16_t h) {
  return (uint16_t)(stream_op2<DT, OP>((uint32_t)h) & 0xffffu);
}

// Chunked kernel: out and in are both contiguous [rows*hidden], 16-byte
// aligned.  Workgroup g moves the UNROLL*BLOCK vectors starting at vector
// g*UNROLL*BLOCK (lane t takes t, t+BLOCK, ...: each wave instruction covers
// 1 KiB), all loads before all stores, non-temporal both ways.  One
// workgroup per chunk, no grid-stride loop.
template <int DT, int OP, int UNROLL, int BLOCK>
// in, out and the vector count lead the arguments, so that gfx950 preloads
// them into SGPRs (the first loads wait for no scalar memory load)
__global__ __launch_bounds__(BLOCK) void stream_chunk_kernel(const uint16_t* in16, uint16_t* out16, int64_t nvec,
                                                             StreamArgs a) {
  const u32x4* in = reinterpret_cast<const u32x4*>(in16);
  u32x4* out = reinterpret_cast<u32x4*>(out16);
  const int64_t base = (int64_t)blockIdx.x * (UNROLL * BLOCK) + threadIdx.x;
  u32x4 v[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + u * BLOCK;
    if (i < nvec) v[u] = __builtin_nontemporal_load(in + i);
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + u * BLOCK;
    if (i < nvec) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = stream_op2<DT, OP>(v[u][j]);
      __builtin_nontemporal_store(o, out + i);
    }
  }
  if (blockIdx.x == gridDim.x - 1) {  // elements past the last whole vector
    const int64_t total = a.rows * a.hidden;
    for (int64_t e = nvec * 8 + threadIdx.x; e < total; e += BLOCK)
      out16[e] = stream_op1<DT, OP>(in16[e]);
  }
}

// Row streamer: any row strides, rows at any 2-byte boundary.  Work unit u =
// (row, chunk): BLOCK lanes, one 16-byte vector each (4 KiB per workgroup, as
// the flat kernel), accesses through buffer resources sized to the row
// (unaligned 16-byte accesses are legal here, see fused_vec_kernel), so the
// range check drops everything past the row's whole vectors (nvec per
// row).  hidden % 8 != 0: the lane holding the last whole vector also moves
// the 16 bytes that end at the row's end; they overlap that vector, whose
// elements it writes again with the same values (both ops are idempotent, so
// this holds in place too).  hidden < 8: the first hidden lanes move one
// element each.
template <int DT, int OP, int BLOCK>
// every field leads as a scalar argument (preloaded into SGPRs on gfx950),
// with the launched grid, which never exceeds rows * chunks
__global__ __launch_bounds__(BLOCK) void stream_rows_kernel(const uint16_t* in16, uint16_t* out16, int64_t rows,
                                                            int64_t in_stride, int64_t out_stride, int32_t hidden,
                                                            int32_t nvec, int32_t grid) {
  const int64_t chunks = nvec > 0 ? (nvec + BLOCK - 1) / BLOCK : 1;
  const uint32_t rowbytes = (uint32_t)hidden * 2u;
  const int tcount = (int)(hidden - nvec * 8);
  for (int64_t u = blockIdx.x; u < rows * chunks; u += grid) {
    const int64_t row = u / chunks;
    const int64_t v = (u - row * chunks) * BLOCK + threadIdx.x;
    const __amdgpu_buffer_rsrc_t irs = make_rsrc(in16 + row * in_stride, rowbytes);
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(out16 + row * out_stride, rowbytes);
    if (nvec == 0) {  // hidden < 8
      const uint32_t off = (uint32_t)threadIdx.x * 2u;
      __builtin_amdgcn_raw_buffer_store_b16(stream_op1<DT, OP>(__builtin_amdgcn_raw_buffer_load_b16(irs, off, 0, 0)),
                                            ors, off, 0, 0);
      continue;
    }
    const bool ok = v < nvec;
    const bool tail = tcount > 0 && v == nvec - 1;
    const uint32_t off = ok ? (uint32_t)v * 16u : kOOB;
    const uint32_t toff = tail ? rowbytes - 16u : kOOB;
    const u32x4 x = load16<kAuxNT>(irs, off);
    const u32x4 t = load16<kAuxNT>(irs, toff);
    u32x4 o, ot;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[j] = stream_op2<DT, OP>(x[j]);
      ot[j] = stream_op2<DT, OP>(t[j]);
    }
    store16<kAuxNT>(o, ors, off);
    store16<kAuxNT>(ot, ors, toff);
  }
}

}  // namespace hprms
