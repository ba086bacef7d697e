"""SLA2 (sparse-linear attention v2) module family on the gfx950 kernels.

Same names as the reference's vendored package (models/sla2_vendor/__init__.py):
SLA2, sla2_dense, full_attention, Router.
"""
from .core import SLA2, full_attention, sla2_dense
from .router import Router
