// Matrix-core (MFMA) tiered decode kernel -- not enabled yet; every format
// runs the portable kernel in decode.hip.
#include "decode_common.h"

namespace fade {
namespace decode {

bool mfma_supports(const Params&) { return false; }
int mfma_tile() { return 64; }
int launch_mfma(const Params& p, hipStream_t st) { return launch_valu(p, st); }

}  // namespace decode
}  // namespace fade
