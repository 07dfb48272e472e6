// Split-KV attention variants with half_t elements (q, y, fp cache, scales).
#define MOTIF_ELEM half_t
#define MOTIF_SUFFIX f16
#include "sdpa_inst.hpp"
