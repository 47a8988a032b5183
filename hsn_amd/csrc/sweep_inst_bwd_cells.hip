// The kernels of the reference-form recurrence (c, b given; int64 cells), instantiated in a
// translation unit of their own so the sweeps' kernels compile in parallel.
#define HSN_SWEEP_INSTANTIATE
#include "sweep.cuh"

namespace hsn {
template hipError_t launch_bwd<float, Cells64, false>(const BwdArgs&, int, size_t, hipStream_t);
}  // namespace hsn
