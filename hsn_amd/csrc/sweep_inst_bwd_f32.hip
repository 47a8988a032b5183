// The kernels of the backward sweep, f32 storage and int32 slots, instantiated in a
// translation unit of their own so the sweeps' kernels compile in parallel.
#define HSN_SWEEP_INSTANTIATE
#include "sweep.cuh"

namespace hsn {
template hipError_t launch_bwd<float, Packed32, true>(const BwdArgs&, int, size_t, hipStream_t);
}  // namespace hsn
