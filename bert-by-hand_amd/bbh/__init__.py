"""MI355X (gfx950) MiniLM-L6 sentence-embedding engine: Python host layer.

``bbh.engine`` mirrors the reference's C++ host API over the C ABI of
``include/bbh.h`` (``libbbh.so``); ``bbh.synth`` makes the seeded synthetic
weights and token batches.  Importing ``bbh.engine`` does not load the
library; the first call does, and raises if it has not been built.
"""

from . import synth  # noqa: F401
