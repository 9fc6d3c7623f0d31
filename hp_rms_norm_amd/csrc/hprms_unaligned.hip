// hprms_unaligned.hip - the vector-tier kernels for rows that do not start on
// 128-byte boundaries (rows at any 2-byte boundary: 16-byte accesses at
// unaligned addresses), hidden % 8 == 0.  One variant of every shape the
// dispatch tables choose, with the same lanes, vectors and weight timing.  In
// modes 0, 1, 3 and 4 the variants rotate each row's lane mapping so that
// every wave's 1 KiB chunk starts on a 512-byte boundary (the kernel's
// rotation phases) and writes whole cache lines, and the shapes with the sc1 policy
// bits also come with them; the FP8 and MX variants, whose chunks share their
// first and last line with the next chunk, go without (such partial lines
// written with sc1 measured 13-24% slower at 16K-32K, 4096 rows, row stride
// hidden + 8).  Kept in its own translation unit so that the build compiles
// it in parallel with hprms.hip; hprms_tail.hip holds the same shapes with
// the tail vector for hidden % 8 != 0.
#include <hip/hip_runtime.h>

#include "hp_rms_norm_amd.h"
#include "hprms_registry.h"

namespace hprms {

const FusedEntry kFusedUnaligned[] = {
    HPRMS_ALL_MODES_OFFGRID(HPRMS_UNALIGNED_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ALL_MODES_OFFGRID(HPRMS_UNALIGNED_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_ROTATED_MODES_SC1(HPRMS_UNALIGNED_SC1_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ROTATED_MODES_SC1(HPRMS_UNALIGNED_SC1_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_MX_MODES(HPRMS_UNALIGNED_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_MX_MODES(HPRMS_UNALIGNED_ENTRY, HPRMS_DTYPE_FP16)
};

const int kFusedUnalignedCount = (int)(sizeof(kFusedUnaligned) / sizeof(kFusedUnaligned[0]));

}  // namespace hprms
