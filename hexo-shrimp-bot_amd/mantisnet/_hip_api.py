"""ctypes signatures of libmantis_hip.so (include/mantis_hip.h)."""

from __future__ import annotations

import ctypes

vp = ctypes.c_void_p
i64 = ctypes.c_int64
i32 = ctypes.c_int32
f32p = ctypes.POINTER(ctypes.c_float)



class MantisSubstage(ctypes.Structure):
    """`mantis_substage` of include/mantis_hip.h: one stage of
    mantis_attention_substages (device pointers, sizes)."""

    _fields_ = [
        ("wq", vp), ("bq", vp), ("k", vp), ("v", vp), ("ldk", i64), ("ldv", i64), ("n_src", i64),
        ("bias", vp), ("n_classes", i64), ("vcls", vp), ("seg_ptr", vp), ("src", vp), ("cls", vp),
        ("n_entries", i64), ("wo", vp), ("bo", vp),
    ]


SIGNATURES = {
    "mantis_hip_version": ([], i32),
    "mantis_plan_check": ([vp, vp, i64, vp, vp, i64, vp, i64, i64, vp, vp], i32),
    "mantis_stable_key_order_workspace": ([i64, i64], i64),
    "mantis_stable_key_count": ([vp, i64, i64, vp, vp, vp], i32),
    "mantis_stable_key_order": ([vp, vp, vp, i64, i64, vp, vp, vp, vp, vp], i32),
    "mantis_stable_key_order_noalloc": ([vp, vp, vp, i64, i64, vp, vp, vp, vp, vp], i32),
    "mantis_latent_read_x_workspace": ([i64], i64),
    "mantis_latent_read_x": ([vp, i64, vp, i64, vp, vp, i64, i64, vp, vp, vp, vp, vp, vp], i32),
    "mantis_latent_broadcast_residual": ([vp, i64, vp, i64, vp, i64, i64, vp, vp, vp, i64, vp, vp], i32),
    "mantis_latent_broadcast_project_residual": ([vp, vp, vp, i64, vp, i64, i64, vp, vp, vp, i64, vp, vp], i32),
    "mantis_covered_rows": ([vp, vp, i64, i64, vp, vp, i64, vp, vp, vp], i32),
    "mantis_window_view": ([vp, vp, vp, vp, i64, i64, i64, vp, vp, i64, vp, vp, vp, vp, vp, vp], i32),
    "mantis_radius_class": ([vp, vp, vp, i64, vp, vp], i32),
    "mantis_attention_slots": ([vp, i64, i64, i64, vp, vp, vp, vp], i32),
    "mantis_gather_rows": ([vp, i32, i64, i64, vp, vp, i64, i64, vp, i64, vp, vp], i32),
    "mantis_runs_to_ptr": ([vp, i64, i64, vp, vp, vp], i32),
    "mantis_structure_init": ([vp, vp, i64, vp, i64, vp, i64, vp, vp, i64, vp, i64, vp, i64, vp, i64, vp, vp], i32),
    "mantis_segment_order": ([vp, i64, vp, vp, i64, vp, vp, vp], i32),
    "mantis_run_reduce": ([vp, i32, i64, i64, i64, vp, i64, vp, i64, vp, i32, vp, vp], i32),
    "mantis_class_reduce_workspace": ([i64, i64, i64], i64),
    "mantis_class_reduce": ([vp, i32, i64, i64, i64, vp, i64, vp, i64, vp, i64, vp, i32, vp, vp], i32),
    "mantis_cell_pass": ([vp, i32, i64, i64, i64, vp, i32, i64, i64, vp, i64, vp, vp, i64, vp, vp, vp, vp, vp, vp],
                         i32),
    "mantis_attention_backward_workspace": ([i64, i64, i64], i64),
    "mantis_attention_backward": ([vp, vp, vp, i32, i64, i64, i64, i64, i64, vp, i64, vp, i32, vp, i64, vp, vp, vp,
                                   vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, vp], i32),
    "mantis_row_encode_backward_workspace": ([i64, i64], i64),
    "mantis_row_encode_backward": ([vp, i32, i64, i64, vp, i32, i64, vp, i64, vp, vp, vp, i64, vp, vp, vp, vp, vp, i64,
                                    vp, vp, vp, vp], i32),
    "mantis_cell_pass_backward_workspace": ([i64, i64, i64, i64], i64),
    "mantis_cell_pass_backward": ([vp, i32, i64, i64, i64, vp, i32, i64, i64, vp, i32, i64, vp, i64, vp, vp, i64, vp,
                                   vp, vp, vp, vp, i64, vp, vp, vp, vp], i32),
    "mantis_cell_attention": (
        [vp, vp, vp, i32, i64, i64, i64, vp, i64, vp, i32, vp, vp, vp, i64, i64, i64, i32, i32, vp, i32, vp, vp, vp, vp],
        i32),
    "mantis_attention_substage": (
        [vp, i64, i64, vp, vp, vp, vp, i64, i64, i64, vp, i64, vp, vp, vp, vp, i64, vp, vp, vp, vp], i32),
    "mantis_attention_substages": ([vp, i32, i64, i64, vp, vp, i32, vp, vp, vp], i32),
    "mantis_attention_substages_init": ([vp, i32, i64, i64, vp, vp, i32, vp, i64, i64, vp, i64, vp, vp, vp], i32),
    "mantis_attention_substages_covered": ([vp, i32, i64, i64, vp, vp, vp, i64, i64, vp, i64, vp, vp, vp], i32),
    "mantis_attention_substage_project": ([vp, i32, i64, i64, vp, vp, vp, vp, vp, i64, vp, vp, vp], i32),
    "mantis_radius_chunks_capacity": ([i64, i64], i64),
    "mantis_radius_chunks": ([vp, vp, i32, i64, i64, i64, vp, i64, vp, vp, vp], i32),
    "mantis_radius_prep": ([vp, vp, i64, vp, i64, vp, vp, i64, i64, i64, vp, i64, vp, i64, vp, vp, vp, vp, vp], i32),
    "mantis_radius_stage": ([vp, i64, i64, vp, vp, vp, i64, vp, vp, vp, vp, i64, i64, vp, i64, vp, vp, i64, vp, vp,
                             vp, vp, i64, i64, vp, vp, vp], i32),
    "mantis_cell_heads": (
        [vp, i32, i32, i32, i64, i64, vp, vp, vp, vp, vp, vp, vp, i64, vp, i64, vp, vp, vp, vp, i64, vp, i64, vp, vp, vp,
         vp, vp, i64, vp, vp, vp, vp], i32),
    "mantis_improve_policy": ([vp, vp, vp, i32, vp, i64, i64, ctypes.c_double, ctypes.c_double, vp, vp, vp, vp, vp, vp],
                              i32),
    "mantis_latent_mix": ([vp, i64, i64, vp, vp, vp, vp, vp], i32),
    "mantis_latent_read": ([vp, vp, vp, i32, i64, i64, i64, vp, vp, i64, i64, i32, i32, vp, vp, vp, vp, vp, vp], i32),
    "mantis_latent_read_workspace": ([i64], i64),
    "mantis_latent_broadcast": ([vp, vp, vp, i32, i64, i64, i64, vp, i64, i64, i32, i32, vp, i32, vp, vp, vp, vp],
                                i32),
    "mantis_row_encode": ([vp, i32, i64, i64, vp, i64, vp, vp, i64, vp, i64, vp, vp, vp, vp, vp], i32),
    "mantis_stone_attention": ([vp, vp, vp, vp, vp, vp, i32, vp, i64, i32, i64, i32, vp, vp, vp, vp, vp], i32),
    "mantis_stone_attention_backward": ([vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, i64, i32, i64, i32, vp,
                                         vp, vp, vp, vp, vp, vp, vp], i32),
    "mantis_latent_attend": ([vp, i32, i64, vp, i64, i64, vp, vp], i32),
    "mantis_stone_attention_schedule_len": ([i64, i32, i64], i64),
    "mantis_stone_attention_schedule": ([vp, i64, i32, i64, vp, vp], i32),
    "mantis_fused_linear": ([vp, i32, i64, vp, i64, i64, i32, vp, i32, i64, vp, vp, vp, i32, vp, i64, vp, vp, i64,
                             i32, vp, vp, i32, i32, vp, i64, vp, vp], i32),
    "mantis_fused_linear_split": ([vp, i32, i64, vp, i64, i64, i32, vp, i32, i64, vp, vp, vp, i32, vp, i64, vp, vp,
                                   i64, i32, vp, vp, i32, i32, vp, i64, vp, vp], i32),
    "mantis_layer_norm": ([vp, i32, i64, i64, vp, vp, vp, i32, i64, vp], i32),
    "mantis_value_read": ([vp, vp, i32, i64, vp, vp, i64, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp], i32),
    "mantis_value_read_workspace": ([i64], i64),
    "mantis_compose_q": ([vp, i64, vp, i64, i64, ctypes.c_float, vp, vp, vp], i32),
    "mantis_compose_q_rows": ([vp, i64, vp, i64, i64, ctypes.c_float, vp, vp, vp, vp], i32),
    "mantis_hex_neighbours": ([vp, vp, i64, i64, vp, vp, vp], i32),
    "mantis_hex_aggregate_linear": ([vp, vp, i64, vp, vp, vp, vp, vp, vp], i32),
}


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib
