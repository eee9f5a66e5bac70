// The one translation unit compiled ahead of time into the tiler-hip gfx950
// code object (clang -x hip --offload-arch=gfx950 --offload-device-only).  Every kernel is an
// extern "C" entry so its symbol is the stable name the entry mapping carries.
#include "reduce.hip"
#include "rows.hip"
#include "rows_long.hip"
#include "rows_strict.hip"
#include "gather.hip"
#include "map.hip"
#include "expr.hip"
#include "fold.hip"
#include "convert.hip"
#include "contract.hip"
#include "contract_general.hip"
#include "dequantize.hip"
