// hprms_tail.hip - the vector-tier kernels for hidden % 8 != 0 (hidden >= 8):
// the unaligned variants of hprms_unaligned.hip plus the tail vector, the
// 16 bytes that end at the row's end, handled by the lane that holds the last
// whole vector.  Modes 0-4 only: the MX outputs need hidden % 32 == 0.
#include <hip/hip_runtime.h>

#include "hp_rms_norm_amd.h"
#include "hprms_registry.h"

namespace hprms {

const FusedEntry kFusedTail[] = {
    HPRMS_ALL_MODES_TAIL(HPRMS_TAIL_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ALL_MODES_TAIL(HPRMS_TAIL_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_ROTATED_MODES_SC1_TAIL(HPRMS_TAIL_SC1_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ROTATED_MODES_SC1_TAIL(HPRMS_TAIL_SC1_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_ALL_MODES_WLDS_TAIL(HPRMS_TAIL_WLDS_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ALL_MODES_WLDS_TAIL(HPRMS_TAIL_WLDS_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_WLDS_TAIL_SC1(HPRMS_TAIL_WLDS_SC1_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_WLDS_TAIL_SC1(HPRMS_TAIL_WLDS_SC1_ENTRY, HPRMS_DTYPE_FP16)
};

const int kFusedTailCount = (int)(sizeof(kFusedTail) / sizeof(kFusedTail[0]));

}  // namespace hprms
