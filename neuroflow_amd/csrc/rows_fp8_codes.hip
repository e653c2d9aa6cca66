// rows_fp8_codes.hip -- row-tile kernel instantiations: FP8, code input.
#include "launch_rows.h"

namespace nfq {

template void launch_rows<true, IN_CODES, OUT_EPI>(const RowsArgs&, int, hipStream_t);
template void launch_rows<true, IN_CODES, OUT_RAW>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
