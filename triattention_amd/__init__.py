"""MI355X (gfx950) implementation of TriAttention's quantized attention path.

Host operators mirror the reference package ``triattention``:
``triattention_amd.kernels.prefill.Prefill`` / ``BandTable``,
``triattention_amd.kernels.decode.DecodeCache``, ``triattention_amd.maps`` and
``triattention_amd.kernels.extension.load_extension`` (the C-ABI kernel
library, include/triattention_amd.h).
"""
