// The one translation unit compiled ahead of time into the tiler-hip gfx950
// code object (hipcc --genco --offload-arch=gfx950).  Every kernel is an
// extern "C" entry so its symbol is the stable name the entry mapping carries.
#include "reduce.hip"
#include "rows.hip"
#include "gather.hip"
#include "map.hip"
#include "contract.hip"
