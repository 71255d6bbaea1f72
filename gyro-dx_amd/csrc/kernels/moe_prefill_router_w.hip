// The prefill router, wide build (constants and layouts as moe_prefill_router.hip): each of the
// four MFMA waves takes two 32-expert column tiles (64 experts) over the group's whole K range,
// so a group covers 32 tokens x 256 experts, splits each staged chunk of token rows over two
// tiles, and stores its logits straight from the accumulators. Grid: (ceil(n / 32),
// ceil(n_expert / 256), S); 512 threads, 144 KB of LDS.
#define RT_PIPELINE moe_prefill_router_w
#define RT_TW 2
#include "moe_prefill_router.hip"
