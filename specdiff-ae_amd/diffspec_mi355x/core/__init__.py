"""Host-side policies of the verification path."""

from .bundle_scheduler import BundleScheduler, TreeDescriptorBuilder, bundle_row_order, bundle_row_order_device  # noqa: F401
