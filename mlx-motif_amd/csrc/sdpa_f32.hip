// Split-KV attention variants with float elements (q, y, fp cache, scales).
#define MOTIF_ELEM float
#define MOTIF_SUFFIX f32
#include "sdpa_inst.hpp"
