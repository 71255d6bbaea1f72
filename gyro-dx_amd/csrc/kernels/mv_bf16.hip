// bf16 rows (the shared expert). See mv_common.h.
#include "mv_common.h"
GD_PIPELINE_NAMED(mv_bf16, 256) { mv_body<MV_BF16>(a); }
