// General tier of the fused add + RMSNorm family: any width, alignment and
// row stride (modes 0-4).  Kept in its own translation unit because it
// instantiates the register-resident kernel for many (block, slots) shapes;
// the build compiles it in parallel with hprms.hip.
//
// Shape choice (measured on MI355X, 4096 bf16 rows, in-place fused op):
//   hidden <= 1024          one wave per row (BLOCK 64), E = ceil(h / 64)
//   1024 < hidden <= 8192   BLOCK 256, E = ceil(h / 256)
//   8192 < hidden <= 16384  BLOCK 1024, E = ceil(h / 1024)
//   hidden > 16384          fused_general_kernel (two passes over the row)
// E is rounded up to the next listed slot count; elements past the row cost
// an issued instruction but no memory traffic (the buffer range check drops
// them).  Smaller blocks keep more rows in flight per CU: at hidden = 2049 a
// 1024-thread row took 19.8 us against 11.2 us for 256 threads.

#include <hip/hip_runtime.h>

#include "hprms_kernels.h"

namespace hprms {
namespace {

// Launches fused_general_reg_kernel<DT, MODE, BLOCK, E> for the first E in
// the list that holds `slots` element slots per thread (the last one holds
// every slot count the caller passes).
template <int DT, int MODE, int BLOCK, int E, int... MORE>
void launch_slots(int64_t slots, const GeneralArgs& a, dim3 grid, hipStream_t stream) {
  if constexpr (sizeof...(MORE) > 0) {
    if (slots > E) {
      launch_slots<DT, MODE, BLOCK, MORE...>(slots, a, grid, stream);
      return;
    }
  }
  fused_general_reg_kernel<DT, MODE, BLOCK, E><<<grid, dim3(BLOCK), 0, stream>>>(a);
}

template <int DT, int MODE>
void launch_mode(const GeneralArgs& a, int64_t grid, hipStream_t stream) {
  const dim3 g((unsigned)grid);
  const int64_t h = a.hidden;
  if (h <= 1024)
    launch_slots<DT, MODE, 64, 1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16>((h + 63) / 64, a, g, stream);
  else if (h <= 8192)
    launch_slots<DT, MODE, 256, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32>((h + 255) / 256, a, g, stream);
  else if (h <= 16384)
    launch_slots<DT, MODE, 1024, 10, 12, 14, 16>((h + 1023) / 1024, a, g, stream);
  else
    fused_general_kernel<DT, MODE><<<g, dim3(256), 0, stream>>>(a);
}

template <int DT>
void launch_dtype(const GeneralArgs& a, int mode, int64_t grid, hipStream_t stream) {
  switch (mode) {
    case 0: launch_mode<DT, 0>(a, grid, stream); break;
    case 1: launch_mode<DT, 1>(a, grid, stream); break;
    case 2: launch_mode<DT, 2>(a, grid, stream); break;
    case 3: launch_mode<DT, 3>(a, grid, stream); break;
    default: launch_mode<DT, 4>(a, grid, stream); break;
  }
}

}  // namespace

void launch_general_kernels(const GeneralArgs& a, int dtype, int mode, int64_t grid, hipStream_t stream) {
  if (dtype == HPRMS_DTYPE_BF16)
    launch_dtype<HPRMS_DTYPE_BF16>(a, mode, grid, stream);
  else
    launch_dtype<HPRMS_DTYPE_FP16>(a, mode, grid, stream);
}

}  // namespace hprms
