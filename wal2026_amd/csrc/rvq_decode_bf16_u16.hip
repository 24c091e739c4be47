// decode kernel instantiations for bf16 activations and 16-bit indices.
#include "rvq_decode_impl.h"

namespace wal {
template hipError_t decode_entry<WAL_BF16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&, int, int,
                                              const void*, int M, const DecodePlan&, hipStream_t);
}  // namespace wal
