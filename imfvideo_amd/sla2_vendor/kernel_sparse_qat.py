"""Re-export of quantize_qkv under the reference's vendored module path
(models/sla2_vendor/kernel_sparse_qat.py:144)."""
from ..kernel_sparse_qat import quantize_qkv  # noqa: F401
