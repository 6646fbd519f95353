"""credit_amd -- MI355X (gfx950) wide-row kernels behind a C-ABI library.

``credit_amd.hip_lib`` binds ``libcredit_hip.so`` (built from
``credit_amd/csrc``) through ctypes; ``credit_amd.workloads`` holds the
workload registry.  See ``include/credit.h`` for the C-ABI.
"""
__version__ = "0.1.0"
