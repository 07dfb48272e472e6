// Split-KV attention variants with bf16_t elements (q, y, fp cache, scales).
#define MOTIF_ELEM bf16_t
#define MOTIF_SUFFIX bf16
#include "sdpa_inst.hpp"
