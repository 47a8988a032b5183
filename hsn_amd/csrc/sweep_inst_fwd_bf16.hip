// The kernels of the forward sweep, bf16 storage and int32 slots, instantiated in a
// translation unit of their own so the sweeps' kernels compile in parallel.
#define HSN_SWEEP_INSTANTIATE
#include "sweep.cuh"

namespace hsn {
template hipError_t launch_fwd<bf16_t, bf16_t, Packed32>(const FwdArgs&, int, size_t, hipStream_t);
}  // namespace hsn
