// Library identity and status strings for the C ABI.
#include "common.h"

extern "C" int oxr_abi_version(void) { return OXR_ABI_VERSION; }

extern "C" const char* oxr_status_string(int status) {
  switch (status) {
    case OXR_OK:
      return "ok";
    case OXR_ERR_INVALID_ARG:
      return "invalid argument (null pointer, negative or inconsistent size)";
    case OXR_ERR_UNSUPPORTED:
      return "unsupported shape for the gfx950 kernels";
    case OXR_ERR_WORKSPACE:
      return "workspace missing or smaller than required";
    case OXR_ERR_SCRATCH_LIMIT:
      return "the shape needs more scratch than the library's static scratch array holds "
             "(see oxr_static_scratch_bytes); use the entry point that takes a workspace";
    default:
      break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

// Self-test of the v_mfma_f32_16x16x32_bf16 operand layout every MFMA kernel
// here assumes: lane l holds A[l % 16][8 * (l / 16) + j] and
// B[8 * (l / 16) + j][l % 16] for j < 8, and receives
// C[4 * (l / 16) + i][l % 16] for i < 4.  a is bf16 [16, 32] row-major, b is
// bf16 [32, 16] row-major, c is fp32 [16, 16] row-major.  One wave.
namespace {
__global__ __launch_bounds__(64) void mfma_layout_probe(const uint16_t* a, const uint16_t* b, float* c) {
  using namespace oxr;
  const int l = threadIdx.x;
  const int r = l % 16, g = l / 16;
  uint32_t av[4], bv[4];
  for (int j = 0; j < 4; ++j) {
    av[j] = (uint32_t)a[r * 32 + 8 * g + 2 * j] | ((uint32_t)a[r * 32 + 8 * g + 2 * j + 1] << 16);
    bv[j] = (uint32_t)b[(8 * g + 2 * j) * 16 + r] | ((uint32_t)b[(8 * g + 2 * j + 1) * 16 + r] << 16);
  }
  u32x4 A = {av[0], av[1], av[2], av[3]};
  u32x4 B = {bv[0], bv[1], bv[2], bv[3]};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma_16x16x32(A, B, acc);
  for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r] = acc[i];
}
}  // namespace

extern "C" int oxr_selftest_mfma_layout(const uint16_t* a, const uint16_t* b, float* c, oxr_stream_t stream) {
  OXR_RETURN_IF(!a || !b || !c, OXR_ERR_INVALID_ARG);
  hipLaunchKernelGGL(mfma_layout_probe, dim3(1), dim3(64), 0, (hipStream_t)stream, a, b, c);
  return OXR_LAUNCH_STATUS();
}
