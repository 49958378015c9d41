"""diffspec_mi355x — MI355X-native (gfx950) tree-verification hot path of DiffSpec.

Module layout mirrors the reference package ``diffspec``:
  runtime.tree_attention     prefix_attention_forward, tree_attention_forward, tree_verify
  runtime.attention_compat   flash_attn_with_kvcache / flash_attn_func contract
  runtime.bundle_verifier    FusedBundleVerifier, PagedBundleVerifier
  core.bundle_scheduler      BundleScheduler, TreeDescriptorBuilder, bundle_row_order,
                             bundle_row_order_device
  draft.tree_verification    verify / verify_new, tree_accept, evaluate_tree
All compute runs in libdsv.so (HIP kernels for gfx950 behind a C ABI).
"""

__version__ = "0.1.0"
