module GraphGPHIPExt

# libgraphgp_hip (include/graphgp_hip.h) as GraphGP.jl's backend for problems on AMD GPUs.
#
# It adds methods to GraphGP's own functions for a problem whose arrays are ROCArrays (the
# result of `to_backend(prob, ROCBackend())`), so existing call sites — and the rrules of
# src/chainrules.jl and src/grad_generate_vals.jl:291-305, which call these functions on
# `_set_vals(prob, vals)` — run on the library unchanged:
#
#   generate, generate_inv, generate_logdet                  (src/orchestrate.jl:19-97)
#   refine_logdet, refine_logdet_terms, refine_inv, refine!, refine   (src/api.jl:24-185)
#   generate_grad_xi, generate_grad_vals                      (src/grad.jl:392-506,
#                                                             src/grad_generate_vals.jl:111-282)
#   refine_logdet_grad_vals, generate_logdet_grad_vals, generate_logdet_and_grad_vals,
#   refine_inv_loss_grad_vals, generate_inv_loss_grad_vals    (src/grad.jl:96-154, 514-715)
#   refine_/generate_logdet_grad_points, refine_/generate_inv_loss_grad_points
#                                                             (src/grad.jl:168-377)
#   refine_logdet_custom, refine_inv_custom                   (src/custom_cuda.jl:7-39; the
#                                                             stateless gphip_* entry points)
#
# The library is dlopen'ed lazily from ENV["GRAPHGP_HIP_LIB"] (or the in-tree build), symbols are
# found by name and called with ccall on device pointers, ordered on AMDGPU.jl's task-local
# stream, and a non-zero status raises with the library's message — the pattern of the
# reference's CUDA glue (ext/GraphGPCUDAExt.jl:15-24, 37, 47).
#
# GraphGPProblem is immutable and rebuilt by `_set_vals` for every new table, so the library's
# problem handle (the repacked graph, created once) is cached per coords array; before each op
# the handle's covariance table is replaced if the problem carries another `vals` array. Every
# method accepts (and ignores) the reference's `backend` keyword.
#
# There is no Julia in the build environment: this file is written, not exercised by the tests.

using GraphGP
using AMDGPU
using Libdl
import GraphGP: GraphGPProblem, npoints, nrefined, nneighbors, ndims_space, nbins,
    generate, generate_inv, generate_logdet, refine_logdet, refine_logdet_terms, refine_inv,
    refine!, refine, generate_grad_xi, generate_grad_vals, refine_logdet_grad_vals,
    generate_logdet_grad_vals, generate_logdet_and_grad_vals, refine_inv_loss_grad_vals,
    generate_inv_loss_grad_vals, refine_logdet_grad_points, generate_logdet_grad_points,
    refine_inv_loss_grad_points, generate_inv_loss_grad_points, refine_logdet_custom,
    refine_inv_custom

const ROCProblem{T} = GraphGPProblem{T, <:ROCMatrix}

# ---- library --------------------------------------------------------------------------------
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

_dtype(::Type{Float32}) = Int32(0)
_dtype(::Type{Float64}) = Int32(1)

# ---- the problem handle, cached per coords array ----------------------------------------------
mutable struct Handle
    h::Ptr{Cvoid}
    neighbors::Any       # the arrays the handle was made from (identity checks)
    offsets::Vector{Int}
    indices::Any
    vals::Any            # the table currently set (identity), or nothing
    cov::Any
end

const HANDLES = WeakKeyDict{Any, Handle}()
const HLOCK = ReentrantLock()

function _destroy(hd::Handle)
    hd.h == C_NULL && return
    ccall(_sym(:ggp_graph_destroy), Cint, (Ptr{Cvoid},), hd.h)
    hd.h = C_NULL
end

function _create(prob::ROCProblem{T}) where {T}
    coords = Array(prob.coords)                                   # (D,N) UInt32, point-major
    nbr0 = Int64.(Array(prob.neighbors)) .- 1                     # (K,M) 0-based, point-major
    offs = Int64.(prob.offsets)            # batch ends: the same numbers as 0-based exclusive ends
    idx = prob.indices === nothing ? C_NULL : Int64.(prob.indices) .- 1
    h = Ref{Ptr{Cvoid}}(C_NULL)
    _check(ccall(_sym(:ggp_graph_create), Cint,
        (Ref{Ptr{Cvoid}}, Ptr{UInt32}, Ptr{Int64}, Ptr{Int64}, Int64, Ptr{Int64}, Int64, Int64,
         Int64, Int32, Cdouble, Int32),
        h, coords, nbr0, offs, length(offs), idx, prob.n0, nneighbors(prob), npoints(prob),
        Int32(ndims_space(prob)), Float64(prob.scale), _dtype(T)), "ggp_graph_create")
    hd = Handle(h[], prob.neighbors, prob.offsets, prob.indices, nothing, nothing)
    finalizer(_destroy, hd)
    return hd
end

function _set_table!(hd::Handle, prob::ROCProblem{T}) where {T}
    if prob.cov === nothing
        hd.vals === prob.vals && hd.cov === nothing && return
        bins = Array{T}(prob.bins); vals = Array{T}(prob.vals)
        _check(ccall(_sym(:ggp_set_cov_iso), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Int64),
            hd.h, bins, vals, length(bins)), "ggp_set_cov_iso")
        hd.vals, hd.cov = prob.vals, nothing
    else
        hd.cov === prob.cov && return
        c = prob.cov
        sb = Array{T}(c.spatial_bins); zb = Array{T}(c.z_bins)
        grid = permutedims(Array{T}(c.grid))   # the library's grid is row-major (n_s, n_z)
        _check(ccall(_sym(:ggp_set_cov_aniso), Cint,
            (Ptr{Cvoid}, Ptr{T}, Int64, Ptr{T}, Int64, Ptr{T}, Cdouble),
            hd.h, sb, length(sb), zb, length(zb), grid, Float64(c.alpha)), "ggp_set_cov_aniso")
        hd.vals, hd.cov = nothing, prob.cov
    end
    return
end

# The handle of `prob`, with its table in place.
function _handle(prob::ROCProblem)
    lock(HLOCK) do
        hd = get(HANDLES, prob.coords, nothing)
        if hd === nothing || hd.neighbors !== prob.neighbors || hd.offsets != prob.offsets ||
           hd.indices != prob.indices
            hd === nothing || _destroy(hd)
            hd = _create(prob)
            HANDLES[prob.coords] = hd
        end
        _set_table!(hd, prob)
        return hd.h
    end
end

_dev(::Type{T}, x::ROCArray{T}) where {T} = x
_dev(::Type{T}, x::AbstractArray) where {T} = ROCArray{T}(x)

# ---- forward ops (original order in and out, as src/orchestrate.jl) --------------------------
function generate(prob::ROCProblem{T}, xi::AbstractVector; kwargs...) where {T}
    x = _dev(T, xi); out = similar(x)
    _check(ccall(_sym(:ggp_generate), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), x, out, _stream()), "ggp_generate")
    return out
end

function generate_inv(prob::ROCProblem{T}, values::AbstractVector; kwargs...) where {T}
    v = _dev(T, values); xi = similar(v)
    _check(ccall(_sym(:ggp_generate_inv), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), v, xi, _stream()), "ggp_generate_inv")
    return xi
end

function _scalar(fn::Symbol, prob::ROCProblem)
    out = Ref{Cdouble}(0)
    _check(ccall(_sym(fn), Cint, (Ptr{Cvoid}, Ref{Cdouble}, Ptr{Cvoid}), _handle(prob), out,
        _stream()), String(fn))
    return out[]
end
generate_logdet(prob::ROCProblem{T}; kwargs...) where {T} = T(_scalar(:ggp_generate_logdet, prob))
refine_logdet(prob::ROCProblem{T}; kwargs...) where {T} = T(_scalar(:ggp_refine_logdet, prob))

# Tree-order ops (src/api.jl).
function refine_logdet_terms(prob::ROCProblem{T}; kwargs...) where {T}
    terms = AMDGPU.zeros(T, nrefined(prob))
    _check(ccall(_sym(:ggp_refine_logdet_terms), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), terms, _stream()), "ggp_refine_logdet_terms")
    return terms
end

function refine_inv(prob::ROCProblem{T}, values::AbstractVector; kwargs...) where {T}
    v = _dev(T, values); xi = AMDGPU.zeros(T, nrefined(prob))
    _check(ccall(_sym(:ggp_refine_inv), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), v, xi, _stream()), "ggp_refine_inv")
    return xi
end

function refine!(values::ROCVector{T}, prob::ROCProblem{T}, xi::AbstractVector; kwargs...) where {T}
    x = _dev(T, xi)
    _check(ccall(_sym(:ggp_refine), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), values, x, _stream()), "ggp_refine")
    return values
end

function refine(prob::ROCProblem{T}, initial_values, xi; kwargs...) where {T}
    values = AMDGPU.zeros(T, npoints(prob))
    copyto!(view(values, 1:prob.n0), _dev(T, initial_values))
    return refine!(values, prob, xi)
end

# ---- adjoints --------------------------------------------------------------------------------
function generate_grad_xi(prob::ROCProblem{T}, vbar::AbstractVector; kwargs...) where {T}
    vb = _dev(T, vbar); out = similar(vb)
    _check(ccall(_sym(:ggp_generate_grad_xi), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cvoid}),
        _handle(prob), vb, out, _stream()), "ggp_generate_grad_xi")
    return out
end

function generate_grad_vals(prob::ROCProblem{T}, xi::AbstractVector, vbar::AbstractVector; kwargs...) where {T}
    x = _dev(T, xi); vb = _dev(T, vbar); dv = AMDGPU.zeros(T, nbins(prob))
    _check(ccall(_sym(:ggp_generate_grad_vals), Cint,
        (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{T}, Ptr{Cvoid}), _handle(prob), x, vb, dv, _stream()),
        "ggp_generate_grad_vals")
    return dv
end

function _vals_and_scalar(fn::Symbol, prob::ROCProblem{T}) where {T}
    dv = AMDGPU.zeros(T, nbins(prob)); s = Ref{Cdouble}(0)
    _check(ccall(_sym(fn), Cint, (Ptr{Cvoid}, Ptr{T}, Ref{Cdouble}, Ptr{Cvoid}),
        _handle(prob), dv, s, _stream()), String(fn))
    return T(s[]), dv
end
refine_logdet_grad_vals(prob::ROCProblem; kwargs...) = _vals_and_scalar(:ggp_refine_logdet_grad_vals, prob)[2]
generate_logdet_grad_vals(prob::ROCProblem; kwargs...) =
    _vals_and_scalar(:ggp_generate_logdet_grad_vals, prob)[2]
generate_logdet_and_grad_vals(prob::ROCProblem; kwargs...) =
    _vals_and_scalar(:ggp_generate_logdet_grad_vals, prob)

function _loss_and_vals(fn::Symbol, prob::ROCProblem{T}, data) where {T}
    d = _dev(T, data); dv = AMDGPU.zeros(T, nbins(prob)); loss = Ref{Cdouble}(0)
    _check(ccall(_sym(fn), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ref{Cdouble}, Ptr{Cvoid}),
        _handle(prob), d, dv, loss, _stream()), String(fn))
    return T(loss[]), dv
end
refine_inv_loss_grad_vals(prob::ROCProblem, values::AbstractVector; kwargs...) =
    _loss_and_vals(:ggp_refine_inv_loss_grad_vals, prob, values)
generate_inv_loss_grad_vals(prob::ROCProblem, data::AbstractVector; kwargs...) =
    _loss_and_vals(:ggp_generate_inv_loss_grad_vals, prob, data)

# d/dpoints: the library's N x D point-major buffer is the reference's (D, N) matrix.
function _points(fn::Symbol, prob::ROCProblem{T}) where {T}
    dp = AMDGPU.zeros(T, ndims_space(prob), npoints(prob))
    _check(ccall(_sym(fn), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{Cdouble}, Ptr{Cvoid}),
        _handle(prob), dp, C_NULL, _stream()), String(fn))
    return dp
end
function _points(fn::Symbol, prob::ROCProblem{T}, data) where {T}
    d = _dev(T, data); dp = AMDGPU.zeros(T, ndims_space(prob), npoints(prob))
    _check(ccall(_sym(fn), Cint, (Ptr{Cvoid}, Ptr{T}, Ptr{T}, Ptr{Cdouble}, Ptr{Cvoid}),
        _handle(prob), d, dp, C_NULL, _stream()), String(fn))
    return dp
end
refine_logdet_grad_points(prob::ROCProblem; kwargs...) = _points(:ggp_refine_logdet_grad_points, prob)
generate_logdet_grad_points(prob::ROCProblem; kwargs...) = _points(:ggp_generate_logdet_grad_points, prob)
refine_inv_loss_grad_points(prob::ROCProblem, values::AbstractVector; kwargs...) =
    _points(:ggp_refine_inv_loss_grad_points, prob, values)
generate_inv_loss_grad_points(prob::ROCProblem, data::AbstractVector; kwargs...) =
    _points(:ggp_generate_inv_loss_grad_points, prob, data)

# ---- the reference's accelerator hooks on the stateless entry points ---------------------------
# refine_logdet_custom / refine_inv_custom (src/custom_cuda.jl:7-39, ext/GraphGPCUDAExt.jl:38-63):
# the same ccall shape, with the integer lattice and scale in place of float positions.
_nbr0(prob) = ROCArray{Int64}(Int64.(Array(prob.neighbors)) .- 1)   # (K, M), 0-based

function refine_logdet_custom(prob::ROCProblem{Float32})
    out = AMDGPU.zeros(Float32, 1)
    nbr = _nbr0(prob)
    _check(ccall(_sym(:gphip_refine_logdet_f32), Cint,
        (Ptr{UInt32}, Cfloat, Ptr{Int64}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32},
         Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
        prob.coords, prob.scale, nbr, prob.bins, prob.vals, out, prob.n0, nneighbors(prob),
        npoints(prob), nbins(prob), ndims_space(prob), _stream()), "gphip_refine_logdet_f32")
    AMDGPU.synchronize()
    return Array(out)[1]
end

function refine_inv_custom(prob::ROCProblem{Float32}, values::AbstractVector)
    v = _dev(Float32, values)
    xi = AMDGPU.zeros(Float32, nrefined(prob))
    nbr = _nbr0(prob)
    _check(ccall(_sym(:gphip_refine_inv_f32), Cint,
        (Ptr{UInt32}, Cfloat, Ptr{Int64}, Ptr{Float32}, Ptr{Float32}, Ptr{Float32},
         Ptr{Float32}, Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
        prob.coords, prob.scale, nbr, prob.bins, prob.vals, v, xi, prob.n0, nneighbors(prob),
        npoints(prob), nbins(prob), ndims_space(prob), _stream()), "gphip_refine_inv_f32")
    AMDGPU.synchronize()
    return xi
end

end # module
