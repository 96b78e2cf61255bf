// The matrix-core GEMM kernels whose wave ranges are staged in windows and
// restaged per tile (long rows at many tokens: a 7B down projection, n_in
// 18944): the MW = true set of orc_mmq_core.hpp, compiled apart from the
// one-window set so the two build in parallel.
#include "orc_mmq_core.hpp"

namespace orc {

int mmq_launch_windowed(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    return mmq_launch_t<true>(type, p, s, ev);
}

}  // namespace orc
