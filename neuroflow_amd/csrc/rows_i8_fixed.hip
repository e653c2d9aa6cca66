// rows_i8_fixed.hip -- row-tile kernel instantiations: INT8, fp32 input with a fixed scale.
#include "launch_rows.h"

namespace nfq {

template void launch_rows<false, IN_F32_FIXED, OUT_EPI>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
