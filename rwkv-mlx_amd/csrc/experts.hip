// Full-expert MoE ChannelMix (rwkv_mlx/moe.py:170-242, MoE_CMix): E
// independent ChannelMix experts, each token sent to its top-k.  The
// reference evaluates every expert on every token and masks (moe.py:223-234);
// here only routed rows are computed:
//   router (router.hip) -> dispatch (dispatch.hip: expert-major positions)
//   -> experts_mix_kernel: row j of perm order, token t = perm[j] / k,
//      expert e = inds[perm[j]]:  xk_j = x[t] + (shift(x)[t] - x[t]) · x_k[e]
//      (model.py:67-75, 260-261, per expert: moe.py:226-227)
//   -> grouped key GEMM, relu² (moe.py:228)  -> grouped value GEMM (moe.py:229)
//   -> combine_kernel with no base: out[t] = Σ_e, ascending, w_e · out_e[t]
//      (moe.py:231-232)
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void experts_mix_kernel(const T* __restrict__ x, const T* __restrict__ xprev,
                                                          const T* __restrict__ mu, const int* __restrict__ perm,
                                                          const int* __restrict__ inds, int nk, int N, int T_, int C,
                                                          int E, int k, T* __restrict__ xk) {
  constexpr int VEC = 16 / sizeof(T);
  const int cpr = C / VEC;
  const size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (id >= (size_t)nk * cpr) return;
  const int j = (int)(id / cpr), c = (int)(id % cpr) * VEC;
  const int a = perm[j];
  const bool ok = a >= 0 && a < N * k;
  const int t = ok ? a / k : 0;
  int e = ok ? inds[a] : 0;
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);  // the forward writes only valid ids
  const int ts = t % T_;
  const u32x4 xv = *(const u32x4*)(x + (size_t)t * C + c);
  const u32x4 pv = ts > 0 ? *(const u32x4*)(x + (size_t)(t - 1) * C + c)
                          : (xprev ? *(const u32x4*)(xprev + (size_t)(t / T_) * C + c) : zero4());
  *(u32x4*)(xk + (size_t)j * C + c) = shift_mix_chunk<T>(xv, pv, *(const u32x4*)(mu + (size_t)e * C + c));
}

}  // namespace

hipError_t launch_experts_mix(int dtype, const void* x, const void* xprev, const void* mu, const int* perm,
                              const int* inds, int N, int T_, int C, int E, int k, void* xk, hipStream_t s) {
  const int nk = N * k;
  const size_t total = (size_t)nk * (C / (dtype == 0 ? 4 : 8));
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(experts_mix_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (const T*)xprev, (const T*)mu, perm,
                       inds, nk, N, T_, C, E, k, (T*)xk);
  });
  return mark(hipGetLastError(), "experts_mix", s);
}

}  // namespace rwkvmoe
