"""MI355X-native implementation of NPA's sphops hot path.

``npa_amd.sphops`` is the drop-in replacement for the reference package
``sphops``; ``npa_amd/csrc`` holds the HIP kernels and the C ABI
(``include/sphops_hip.h``) they are exported through.
"""
