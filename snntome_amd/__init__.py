"""snntome_amd — MI355X-native (gfx950) SNNtome wave executor.

The product is libk44wavec.so (HIP kernels + host plan compiler + the wavec C ABI,
declared in include/k44wavec.h) and its ctypes binding `snntome_amd.wavec`, which keeps the
reference's wavec.py API.  `snntome_amd.synth` generates the benchmark workloads.
"""

__all__ = ["wavec", "synth"]
