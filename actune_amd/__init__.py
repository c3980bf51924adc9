"""actune_amd: MI355X (gfx950) group-64 packed-integer linear backend.

HIP kernels behind a C ABI (include/actune_hip.h, lib/libactune_hip.so) with
the module surface of ActTune's grouped backend:

    from actune_amd.layers import install_bank, ResidentLinear
    from actune_amd.precision import precision_profile, SharedBank
    from actune_amd.kernels.grouped import GroupedLinear, GroupedPaddedLinear
    from actune_amd.graph import GraphReplay
"""
__version__ = "0.1.0"
