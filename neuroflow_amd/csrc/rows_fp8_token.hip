// rows_fp8_token.hip -- row-tile kernel instantiations: FP8, fp32 input with per-token scales.
#include "launch_rows.h"

namespace nfq {

template void launch_rows<true, IN_F32_TOKEN, OUT_EPI>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
