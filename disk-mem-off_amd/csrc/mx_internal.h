// Declarations shared between the translation units of libmoe_mi355x.so (not exported).
#pragma once

#include "moe_mi355x.h"

// Number of H-slices the router logit kernel uses for this shape.
int mx_router_splits_for(int tokens, int hidden, int e1);

// Upper bound of the m-tile list for `tokens` tokens at m_blk rows per tile.
int mx_max_mtiles(int tokens, int top_k, int n_experts, int has_shared, int m_blk);

// Rows per m-tile the expert kernels use for `tokens` tokens.
int mx_m_blk_for(int tokens, int weight_dtype);
