// prefill kernel instantiations for bf16 activations and 16-bit indices.
#include "rvq_prefill_impl.h"

namespace wal {
template hipError_t prefill_entry<WAL_BF16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&, int, int,
                                              const void*, int64_t M, int shape, const PrefillSplit&, hipStream_t);
}  // namespace wal
