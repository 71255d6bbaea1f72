// fp32 rows (the router, the shared-expert gate vector). See mv_common.h.
#include "mv_common.h"
GD_PIPELINE_NAMED(mv_f32, 256) { mv_body<MV_F32>(a); }
