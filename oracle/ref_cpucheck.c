/* ref_cpucheck.c -- compiled without ISA flags so it can run on any x86-64
 * host: reports whether this CPU can execute the AVX-512/VNNI code the
 * reference kernels in libwmref.so were compiled to.  Test infrastructure only. */
__attribute__((visibility("default"))) int ref_cpu_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx512f") &&
           __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") &&
           __builtin_cpu_supports("avx512vnni");
}
