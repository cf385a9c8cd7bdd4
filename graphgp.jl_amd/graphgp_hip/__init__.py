"""graphgp_hip — GraphGP.jl's fused per-point Vecchia refinement on MI355X (gfx950).

The public names mirror GraphGP.jl's exports (src/GraphGP.jl:27-57) for the refinement path:
problem container and backend move, the forward ops, their adjoints, the tables and the graph
build. The computation runs in libgraphgp_hip.so (C ABI: include/graphgp_hip.h); this package is
the host-side binding. The rrules live in graphgp_hip.autograd (imported on demand; needs torch).
"""
from ._native import GraphGPError, build
from .extras import hyperparam_grad, make_cov_bins, matern_kernel, rbf_kernel
from .graph import (build_graph, build_graph_arrays, build_graph_device_arrays, load_graph,
                    save_graph)
from .problem import (
    AnisoCov,
    GraphGPProblem,
    build_anisotropic_covariance,
    HipProblem,
    check_graph,
    generate,
    generate_grad_vals,
    generate_grad_xi,
    generate_inv,
    generate_inv_loss_grad_points,
    generate_inv_loss_grad_vals,
    generate_logdet,
    generate_logdet_and_grad_points,
    generate_logdet_and_grad_vals,
    generate_logdet_grad_points,
    generate_logdet_grad_vals,
    nbins,
    ndims_space,
    nneighbors,
    npoints,
    nrefined,
    refine,
    refine_inv,
    refine_inv_loss_grad_points,
    refine_inv_loss_grad_vals,
    refine_logdet,
    refine_logdet_grad_points,
    refine_logdet_grad_vals,
    refine_logdet_terms,
    to_backend,
)

__all__ = [n for n in dir() if not n.startswith("_")]
