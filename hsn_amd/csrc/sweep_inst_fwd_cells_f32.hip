// The kernels of the per-position end of round, f32 products and the reference's int64 cells, instantiated in a
// translation unit of their own so the sweeps' kernels compile in parallel.
#define HSN_SWEEP_INSTANTIATE
#include "sweep.cuh"

namespace hsn {
template hipError_t launch_fwd<float, float, Cells64>(const FwdArgs&, int, size_t, hipStream_t);
}  // namespace hsn
