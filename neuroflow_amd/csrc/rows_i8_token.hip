// rows_i8_token.hip -- row-tile kernel instantiations: INT8, fp32 input with per-token scales.
#include "launch_rows.h"

namespace nfq {

template void launch_rows<false, IN_F32_TOKEN, OUT_EPI>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
