"""MI355X (gfx950) backend for tinygrad's packed low-bit matmul path.

Importing the package registers the ``MI355X`` device without opening hardware,
as importing tinygrad_dx12 registers DX12 (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/__init__.py:8-10).
"""

from tinygrad_mi355x.compat import register as register

register()
