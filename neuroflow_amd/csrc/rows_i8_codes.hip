// rows_i8_codes.hip -- row-tile kernel instantiations: INT8, code input.
#include "launch_rows.h"

namespace nfq {

template void launch_rows<false, IN_CODES, OUT_EPI>(const RowsArgs&, int, hipStream_t);
template void launch_rows<false, IN_CODES, OUT_RAW>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
