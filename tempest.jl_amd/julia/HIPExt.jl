# HIPExt: Tempest's MI355X target over libtempest_hip, as a package extension.
#
# The Julia side a Tempest maintainer adds to put the HIP backend behind
# `compile`: a `HIPTarget` implementing the Target protocol
# (src/Compiler/runtime/target.jl) and three libraries implementing the
# Implement interface (src/Compiler/Implement/library.jl): products,
# attention and the fused row programs.  Every device operation is a `ccall`
# into libtempest_hip (include/tempest_hip.h); a non-zero status becomes an
# exception, which the cover catches to fall back to its next option
# (src/Compiler/cover/choose.jl:1014-1025).
#
# No Julia toolchain exists where this backend was built, so this file has not
# been run; the same calls, argument for argument, are exercised by the
# Python host in tempest.jl_amd/tempest_hip and its tests.
module HIPExt

using Tempest
import Tempest.Compiler: allocate, upload, upload!, download!, bindable, pointable, capture, recapture, retarget!,
    replay, release, device_name, toolchain, measurable, time_launch, device_rates, quiesce
using Tempest.Compiler.Implement: Library, Template, Binding, Strided
import Tempest.Compiler.Implement: templates, supports, build, repoints, repoint!, loaded

const LIB = get(ENV, "TEMPEST_HIP_LIBRARY", joinpath(@__DIR__, "..", "libtempest_hip.so"))

function check(status::Cint, what)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:th_last_error, LIB), Cstring, ()))
    throw(ErrorException("$what failed ($status): $msg"))
end

# ---- the target ---------------------------------------------------------------------

struct HIPTarget <: Tempest.Compiler.Target
    implementations::Tuple
    device::Int
end

function HIPTarget(implementations...; device::Integer = 0)
    check(ccall((:th_init, LIB), Cint, (Cint,), device), "th_init")
    HIPTarget(implementations, device)
end

"A device buffer: its address and bytes, freed when collected."
mutable struct HIPBuffer{T}
    ptr::Ptr{Cvoid}
    n::Int
    function HIPBuffer{T}(n::Integer) where {T}
        out = Ref{Ptr{Cvoid}}()
        check(ccall((:th_alloc, LIB), Cint, (Csize_t, Ptr{Ptr{Cvoid}}), n * sizeof(T), out), "th_alloc")
        b = new{T}(out[], n)
        finalizer(x -> ccall((:th_free, LIB), Cint, (Ptr{Cvoid},), x.ptr), b)
    end
end
Base.length(b::HIPBuffer) = b.n
Base.eltype(::HIPBuffer{T}) where {T} = T

allocate(::HIPTarget, T, n) = HIPBuffer{T}(n)
upload(t::HIPTarget, x::Array) = upload!(t, allocate(t, eltype(x), length(x)), x)
upload!(::HIPTarget, b::HIPBuffer, x::Array) =
    (check(ccall((:th_upload, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t), b.ptr, x, sizeof(x)), "th_upload"); b)
download!(::HIPTarget, x::Array, b::HIPBuffer) =
    (check(ccall((:th_download, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t), x, b.ptr, sizeof(x)), "th_download"); x)
bindable(::HIPTarget, x) = x isa HIPBuffer
pointable(::HIPTarget, x, at) = x isa HIPBuffer && at % 16 == 0
quiesce(::HIPTarget) = check(ccall((:th_quiesce, LIB), Cint, ()), "th_quiesce")

"One claim's launch: a th_launch* and the buffers it reads, kept alive."
mutable struct HIPLaunch
    handle::Ptr{Cvoid}
    buffers::Vector{Any}
    function HIPLaunch(h, buffers)
        l = new(h, buffers)
        finalizer(x -> ccall((:th_launch_destroy, LIB), Cint, (Ptr{Cvoid},), x.handle), l)
    end
end
(l::HIPLaunch)() = check(ccall((:th_launch_run, LIB), Cint, (Ptr{Cvoid},), l.handle), "th_launch_run")
repoints(::HIPLaunch) = true
function repoint!(l::HIPLaunch, value, buffer::HIPBuffer)
    check(ccall((:th_launch_repoint, LIB), Cint, (Ptr{Cvoid}, Cint, Ptr{Cvoid}), l.handle, value - 1, buffer.ptr),
        "th_launch_repoint")
    l
end

"A captured run of steps: a th_graph* and the launches it keeps."
mutable struct HIPGraph
    handle::Ptr{Cvoid}
    keep::Any
end

function capture(::HIPTarget, steps, keep)
    handles = Ptr{Cvoid}[s.step.run.handle for s in steps]
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_graph_capture, LIB), Cint, (Ptr{Ptr{Cvoid}}, Cint, Ptr{Ptr{Cvoid}}), handles, length(handles), out),
        "th_graph_capture")
    HIPGraph(out[], keep)
end
recapture(t::HIPTarget, g::HIPGraph, steps, keep) = (release(t, g); capture(t, steps, keep))
replay(::HIPTarget, g::HIPGraph) = check(ccall((:th_graph_replay, LIB), Cint, (Ptr{Cvoid},), g.handle), "th_graph_replay")
release(::HIPTarget, g::HIPGraph) =
    (g.handle == C_NULL || ccall((:th_graph_release, LIB), Cint, (Ptr{Cvoid},), g.handle); g.handle = C_NULL; nothing)

# Our kernels' argument layouts are known: the launch is repointed, then its
# graph nodes take its arguments in place; nothing is learned or re-recorded.
function retarget!(::HIPTarget, g::HIPGraph, steps, moves, repoint)
    repoint()
    for (i, s) in enumerate(steps)
        check(ccall((:th_graph_retarget, LIB), Cint, (Ptr{Cvoid}, Cint), g.handle, i - 1), "th_graph_retarget")
    end
    true
end

function device_name(::HIPTarget)
    buf = Vector{UInt8}(undef, 512)
    check(ccall((:th_device_name, LIB), Cint, (Ptr{UInt8}, Csize_t), buf, length(buf)), "th_device_name")
    unsafe_string(pointer(buf))
end

function toolchain(::HIPTarget)
    buf = Vector{UInt8}(undef, 1024)
    check(ccall((:th_toolchain, LIB), Cint, (Ptr{UInt8}, Csize_t), buf, length(buf)), "th_toolchain")
    [Pair(split(kv, "=")...) for kv in split(unsafe_string(pointer(buf)), ";")]
end

measurable(::HIPTarget) = true

function time_launch(::HIPTarget, l::HIPLaunch)
    s = Ref{Cdouble}()
    check(ccall((:th_time_launch, LIB), Cint, (Ptr{Cvoid}, Cint, Ptr{Cdouble}), l.handle, 0, s), "th_time_launch")
    s[]
end

struct Rates
    launch::Cdouble
    cached::Cdouble
    bandwidth::Cdouble
    cache::Cdouble
    blocks::Cdouble
end

function device_rates(::HIPTarget)
    r = Ref{Rates}()
    check(ccall((:th_device_rates, LIB), Cint, (Ptr{Rates},), r), "th_device_rates")
    (launch = r[].launch, cached = r[].cached, bandwidth = r[].bandwidth, cache = r[].cache, blocks = r[].blocks)
end

# ---- products (replaces cuBLASProducts, ext/cuBLASExt.jl) ---------------------------------

struct HIPProducts <: Library end
loaded(::Type{HIPProducts}) = true

product(A, B) = Tempest.Compiler.contract(A, B, (1, 3), (3, 2), (1, 2))
const PRODUCTS = (Template(product; inputs = (A = (:m, :k), B = (:k, :n)), outputs = (:C,)),)
templates(::HIPProducts, ::HIPTarget) = PRODUCTS

struct GemmDesc
    m::Int32; n::Int32; k::Int32; c_dtype::Int32; epilogue::Int32; reserved::Int32
    a::Ptr{Cvoid}; a_m::Int64; a_k::Int64
    b::Ptr{Cvoid}; b_k::Int64; b_n::Int64
    c::Ptr{Cvoid}; c_ld::Int64
    bias::Ptr{Cvoid}; aux::Ptr{Cvoid}; aux_ld::Int64; aux_out::Ptr{Cvoid}; row_sums::Ptr{Cvoid}; loss::Ptr{Cvoid}
end

# bf16 factors, a unit stride on each operand, the result column-major.
function supports(::HIPProducts, ::HIPTarget, b::Binding)
    A, B, C = b.arrays.A, b.arrays.B, b.arrays.C
    A.eltype === B.eltype === Tempest.BFloat16 || return false
    1 in A.strides && 1 in B.strides && C.strides[1] == 1 || return false
    all(s -> s % 8 == 0, (b.extents.m, b.extents.n, b.extents.k))
end

address(s::Strided) = s.buffer.ptr + s.offset * sizeof(s.eltype)

function build(::HIPProducts, ::HIPTarget, b::Binding, resources)
    A, B, C = b.arrays.A, b.arrays.B, b.arrays.C
    d = Ref(GemmDesc(b.extents.m, b.extents.n, b.extents.k, C.eltype === Float32 ? 0 : 1, 0, 0,
        address(A), A.strides[1], A.strides[2], address(B), B.strides[1], B.strides[2], address(C), C.strides[2],
        C_NULL, C_NULL, 0, C_NULL, C_NULL, C_NULL))
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_gemm, LIB), Cint, (Ptr{GemmDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_gemm")
    (HIPLaunch(out[], Any[A.buffer, B.buffer, C.buffer]), "MFMA bf16 product $(b.extents.m)×$(b.extents.n) summing $(b.extents.k)")
end

# ---- attention (replaces cuDNNAttention, ext/cuDNNExt.jl, and the cuTile sweep) ----------

struct HIPAttention <: Library end
loaded(::Type{HIPAttention}) = true

# The forward as test/fixtures/operations.jl writes it; the backward's
# template is its gradient, which the same kernels' backward realizes.
attention_causal(q, k, v) = Tempest.attention(q, k, v; causal = true)
const ATTENTION = (Template(attention_causal; inputs = (q = (:d, :h, :m, :b), k = (:d, :h, :n, :b), v = (:d, :h, :n, :b)),
    outputs = (:o,)),)
templates(::HIPAttention, ::HIPTarget) = ATTENTION

supports(::HIPAttention, ::HIPTarget, b::Binding) =
    b.arrays.q.eltype === Tempest.BFloat16 && b.extents.d == 128 && b.extents.m % 128 == 0 && b.arrays.q.strides[1] == 1

# th_build_attention_fwd / th_build_attention_bwd take a th_attention_desc
# with the strides of q (heads, positions, batch) and k; see include/tempest_hip.h.

# ---- the fused row programs (the cuTile resident sketch for these folds) -----------------

struct HIPRows <: Library end
loaded(::Type{HIPRows}) = true

softmax_grad(x, g) = (y = exp.(x .- Tempest.logsumexp(x; dims = 1)); y .* (g .- sum(y .* g; dims = 1)))
const ROWS = (Template(softmax_grad; inputs = (x = (:n, :r), g = (:n, :r)), outputs = (:dx,)),)
templates(::HIPRows, ::HIPTarget) = ROWS
supports(::HIPRows, ::HIPTarget, b::Binding) = b.arrays.x.eltype === Float32 && b.arrays.x.strides[1] == 1

function build(::HIPRows, ::HIPTarget, b::Binding, resources)
    x, g, dx = b.arrays.x, b.arrays.g, b.arrays.dx
    loss = HIPBuffer{Float32}(1)
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_softmax_grad, LIB), Cint,
        (Int64, Int32, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Ptr{Cvoid}}),
        b.extents.r, b.extents.n, x.strides[2], address(x), address(g), address(dx), loss.ptr, out), "th_build_softmax_grad")
    (HIPLaunch(out[], Any[x.buffer, g.buffer, dx.buffer, loss]), "fused softmax gradient, rows resident")
end

end # module
