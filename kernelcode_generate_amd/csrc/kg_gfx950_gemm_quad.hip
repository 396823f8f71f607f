// Translation unit of one kernel family of libkg_gfx950.so: the explicit instantiations
// kg_gfx950/instances.h lists for it (compiled in parallel with the other families).
#define KG_INSTANTIATE
#define KG_INSTANTIATE_GEMM_QUAD
#include "kg_gfx950/instances.h"
