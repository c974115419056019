"""MI355X-native Kokoro-82M iSTFTNet decoder forward + backward.

The product is the C-ABI shared library built from ``csrc/`` (HIP kernels for
gfx950 plus the C++ drop-in layer for ``kokoro_decoder_backward.h``); this
package holds its ctypes binding (``native``), the decoder configurations
(``config``) and the deterministic synthetic-data generator (``synth``).
"""
