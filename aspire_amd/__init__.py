"""MI355X (gfx950) implementation of ASPIRE's mixed draft/verify paged-KV attention path.

Modules mirror the reference package layout so that call sites switch by import
path (``aspire.attention.kv_ops`` -> ``aspire_amd.attention.kv_ops`` and so on):

``aspire_amd.attention.kv_ops``           ``mylib::update_kv_padded`` / ``mylib::update_kv``
``aspire_amd.attention.page_list``        ``build_unified_indices``
``aspire_amd.attention.holistic_wrapper`` ``HolisticAttentionWrapper``, ``build_holistic_dump_jit_args``
``aspire_amd.attention.flashinfer``       ``validate_flashinfer_patch``, ``compute_max_cta_tile_kv``
``aspire_amd.backends.page_selector``     ``PageSelector``, ``PageSelectorFirstLastAvg``, ``KeyMeanPageSelector``
``aspire_amd.backends.jit_kernels``       ``build_dump_struct``, ``build_dump_jit_args``

All device work runs in libaspire_hip.so (hand-written HIP for gfx950) through
the C ABI in ``include/aspire_hip.h``.
"""

__version__ = "0.1.0"
