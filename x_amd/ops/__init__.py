"""Event-transport ops (splat, gather, anchored pair sums) with the API of the reference's atl.ops."""
from .functional import (PairPlan, anchored_log_scores, anchored_score_mean, ats_pair_sums, ats_pair_sums_flow,
                         ats_pair_sums_traj,
                         blur, build_pair_plan,
                         event_noise, gather, gaussian_kernel1d, image_variance, knn_indices, layout_scope, pair_counts, sample_grid_hip, splat,
                         traj_displacement, traj_origin, traj_visible_fraction, visible_fraction_linear, voxel_grid, warp_splat_gather, window_counts)
from ._ext import ext_supports, get_ext

__all__ = ["splat", "gather", "blur", "gaussian_kernel1d", "ats_pair_sums", "ats_pair_sums_flow", "ats_pair_sums_traj", "build_pair_plan", "PairPlan",
           "window_counts", "voxel_grid", "get_ext", "ext_supports", "pair_counts", "sample_grid_hip",
           "traj_displacement", "traj_origin", "traj_visible_fraction", "visible_fraction_linear", "anchored_log_scores", "anchored_score_mean", "event_noise", "knn_indices", "layout_scope",
           "warp_splat_gather", "image_variance"]
