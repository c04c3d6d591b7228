// host_cpu.cc -- the host CPU's distance kernel sets (host-only code).
//
// vdb picks its distance kernels from the CPU it runs on (src/distance/cpu_features.cc:
// 19-21, 40-48): scalar always, AVX2 with AVX2 + FMA, AVX-512 with AVX-512F on top.  The GPU
// reproduces the arithmetic order of whichever set a vdb process on this host would use.

namespace vdbg {

// 0 = scalar, 1 = avx2, 2 = avx512.
int BestHostKernelSet() {
  __builtin_cpu_init();
  const bool avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  if (avx2 && __builtin_cpu_supports("avx512f")) return 2;
  return avx2 ? 1 : 0;
}

}  // namespace vdbg
