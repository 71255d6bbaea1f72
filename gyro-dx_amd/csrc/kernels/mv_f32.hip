// fp32 rows (the router, the shared-expert gate vector). See mv_common.h.
#include "mv_common.h"
GD_PIPELINE(256) { mv_body<false>(a); }
