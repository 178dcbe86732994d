// The f16-operand (mixed profile) scan kernels.  Built as a separate unit so
// that its MFMA accumulators can be kept in VGPRs (see the Makefile): the
// recurrence wave applies VALU work to its state every chunk, which would
// otherwise cost an AGPR read and write per element.
#include "delta_scan_kernels.hpp"

namespace clef {

int scan_launch_f16(const ScanParams& p, hipStream_t stream) {
  return p.dtype_qkv == 0 ? launch_it<half_t, float>(p, stream) : launch_it<half_t, half_t>(p, stream);
}

}  // namespace clef
