"""The one supported backend configuration (mirrors DELTA/Engine/DELTA/public_config.py:9-20).

Same keys and values as the reference's FINAL_PUBLIC_DELTA_BACKEND_CONFIG, so
``LMBackend(**FINAL_PUBLIC_DELTA_BACKEND_CONFIG)`` works unchanged.  On this
build the planner scoring and selection run inside the captured decode step,
so ``cuda_graph_delta_subset_segments`` (segmenting the graph around an eager
planner) and ``delta_subset_plan_reuse`` (FlashInfer host-plan reuse) are
accepted for compatibility and have nothing left to switch.
"""

FINAL_PUBLIC_DELTA_BACKEND_CONFIG = {
    "page_selector_version": "v2",
    "delta_dump_buffer_dtype": "fp32",
    "delta_page_score_impl": "del3_legacy_softmax",
    "cuda_graph_delta_subset_segments": True,
    "delta_fused_page_scores": True,
    "delta_fixed_selector": True,
    "delta_fast_decode_page_info": True,
    "delta_v2_position_bias": True,
    "delta_subset_plan_reuse": True,
    "delta_impl_profile": False,
}
