module GraphGPHIPExt

# Binding of libgraphgp_hip (include/graphgp_hip.h) for GraphGP.jl on AMD GPUs, in the pattern of
# the reference's CUDA accelerator glue (ext/GraphGPCUDAExt.jl:15-24, 37, 47): the library is
# dlopen'ed lazily from ENV["GRAPHGP_HIP_LIB"] (or the in-tree build), symbols are looked up by
# name and called with ccall on device pointers, ordered on AMDGPU.jl's stream, and a non-zero
# status raises with the library's message. Written against GraphGP.jl's types; there is no Julia
# in the build environment, so this file is not exercised by the test suite.

using GraphGP
using AMDGPU
using Libdl
import GraphGP: GraphGPProblem, npoints, nrefined, nneighbors, ndims_space, nbins

const LIBREF = Ref{Ptr{Cvoid}}(C_NULL)
function _lib()
    LIBREF[] != C_NULL && return LIBREF[]
    path = get(ENV, "GRAPHGP_HIP_LIB", joinpath(@__DIR__, "..", "libgraphgp_hip.so"))
    isfile(path) || error("libgraphgp_hip not found at $path — build it with " *
                          "`make -C graphgp.jl_amd/csrc` (or set ENV[\"GRAPHGP_HIP_LIB\"]).")
    LIBREF[] = Libdl.dlopen(path)
    return LIBREF[]
end
_sym(name) = Libdl.dlsym(_lib(), name)
_stream() = AMDGPU.stream().stream   # hipStream_t of the task-local stream

function _check(rc, fn)
    rc == 0 && return nothing
    msg = unsafe_string(ccall(_sym(:ggp_last_error), Cstring, ()))
    error("$fn returned $rc: $msg")
end

# A device problem: the handle owns the device copies (the analogue of to_backend).
mutable struct HIPProblem{T}
    h::Ptr{Cvoid}
    prob::GraphGPProblem
end

function hip_problem(prob::GraphGPProblem{T}) where {T}
    coords = Array(prob.coords)                                   # (D,N) UInt32, point-major
    nbr0 = Int64.(Array(prob.neighbors)) .- 1                     # (K,M) 0-based, point-major
    offs = Int64.(prob.offsets)                                   # 0-based exclusive ends
    idx = prob.indices === nothing ? C_NULL : Int64.(prob.indices) .- 1
    dtype = T === Float32 ? Int32(0) : Int32(1)
    h = Ref{Ptr{Cvoid}}(C_NULL)
    _check(ccall(_sym(:ggp_graph_create), Cint,
        (Ref{Ptr{Cvoid}}, Ptr{UInt32}, Ptr{Int64}, Ptr{Int64}, Int64, Ptr{Int64}, Int64, Int64,
         Int64, Int32, Cdouble, Int32),
        h, coords, nbr0, offs, length(offs), idx, prob.n0, nneighbors(prob), npoints(prob),
        Int32(ndims_space(prob)), Float64(prob.scale), dtype), "ggp_graph_create")
    bins = Array{T}(prob.bins); vals = Array{T}(prob.vals)
    _check(ccall(_sym(:ggp_set_cov_iso), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Int64),
        h[], bins, vals, length(bins)), "ggp_set_cov_iso")
    hp = HIPProblem{T}(h[], prob)
    finalizer(p -> ccall(_sym(:ggp_graph_destroy), Cint, (Ptr{Cvoid},), p.h), hp)
    return hp
end

# generate (src/orchestrate.jl:19-42): original order in and out.
function generate_hip(hp::HIPProblem{T}, xi::ROCVector{T}) where {T}
    out = similar(xi)
    _check(ccall(_sym(:ggp_generate), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        hp.h, xi, out, _stream()), "ggp_generate")
    return out
end

# generate_grad_xi (src/grad.jl:392-506).
function generate_grad_xi_hip(hp::HIPProblem{T}, vbar::ROCVector{T}) where {T}
    out = similar(vbar)
    _check(ccall(_sym(:ggp_generate_grad_xi), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        hp.h, vbar, out, _stream()), "ggp_generate_grad_xi")
    return out
end

# generate_grad_vals (src/grad_generate_vals.jl:111-282).
function generate_grad_vals_hip(hp::HIPProblem{T}, xi::ROCVector{T}, vbar::ROCVector{T}) where {T}
    dv = AMDGPU.zeros(T, nbins(hp.prob))
    _check(ccall(_sym(:ggp_generate_grad_vals), Cint,
        (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{T}, Ptr{Cvoid}), hp.h, xi, vbar, dv, _stream()),
        "ggp_generate_grad_vals")
    return dv
end

# generate_logdet and its fused gradient (src/orchestrate.jl:89-97, src/grad.jl:680-715).
function generate_logdet_hip(hp::HIPProblem)
    out = Ref{Cdouble}(0)
    _check(ccall(_sym(:ggp_generate_logdet), Cint, (Ptr{Cvoid}, Ref{Cdouble}, Ptr{Cvoid}),
        hp.h, out, _stream()), "ggp_generate_logdet")
    return out[]
end

function generate_logdet_and_grad_vals_hip(hp::HIPProblem{T}) where {T}
    dv = AMDGPU.zeros(T, nbins(hp.prob))
    ld = Ref{Cdouble}(0)
    _check(ccall(_sym(:ggp_generate_logdet_grad_vals), Cint,
        (Ptr{Cvoid}, Ptr{T}, Ref{Cdouble}, Ptr{Cvoid}), hp.h, dv, ld, _stream()),
        "ggp_generate_logdet_grad_vals")
    return ld[], dv
end

# generate_logdet_grad_points (src/grad.jl:242-247): the (D, N) matrix the reference returns is
# the library's N x D point-major buffer.
function generate_logdet_grad_points_hip(hp::HIPProblem{T}) where {T}
    dp = AMDGPU.zeros(T, ndims_space(hp.prob), npoints(hp.prob))
    _check(ccall(_sym(:ggp_generate_logdet_grad_points), Cint,
        (Ptr{Cvoid}, Ptr{T}, Ptr{Cdouble}, Ptr{Cvoid}), hp.h, dp, C_NULL, _stream()),
        "ggp_generate_logdet_grad_points")
    return dp
end

# generate_inv_loss_grad_points (src/grad.jl:368-377); data in the original order.
function generate_inv_loss_grad_points_hip(hp::HIPProblem{T}, data::ROCVector{T}) where {T}
    dp = AMDGPU.zeros(T, ndims_space(hp.prob), npoints(hp.prob))
    _check(ccall(_sym(:ggp_generate_inv_loss_grad_points), Cint,
        (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cdouble}, Ptr{Cvoid}), hp.h, data, dp, C_NULL,
        _stream()), "ggp_generate_inv_loss_grad_points")
    return dp
end

end # module
