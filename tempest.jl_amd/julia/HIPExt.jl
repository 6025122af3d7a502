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

# ---- the floor: any pointwise or reduction group, generated ---------------------------
#
# The reference's floor turns a group into Julia code (scalar_kernel,
# src/Compiler/codegen/scalar.jl:186-250) and CUDA compiles it (floor_launch,
# ext/CUDAExt.jl:926-937).  Here the group's terms cross the C ABI as arrays
# (th_floor_desc) and libtempest_hip writes and compiles the gfx950 kernel.
# Supported: Var atoms in addresses, up to two Div or Mod atoms of positions
# and one Indirect atom (a gathered index; other forms throw and the build
# falls back), the functions of FLOOR_FN, and the folds of FLOOR_FOLD.

struct FloorValue; dtype::Int32; reserved::Int32; length::Int64; ptr::Ptr{Cvoid}; end
struct CPart; kind::Int32; reserved::Int32; divisor::Int64; coeff::Int64; constant::Int64; inner::NTuple{4, Int64}; end
struct CAffine
    constant::Int64; coeff::NTuple{4, Int64}; gather::Int32; reserved::Int32; gather_coeff::Int64
    part::NTuple{2, CPart}
end
const NO_PART = CPart(0, 0, 1, 0, 0, (0, 0, 0, 0))
struct CTerm; op::Int32; fn::Int32; args::NTuple{3, Int32}; ref::Int32; observe::Int32; lit::Float32; index::CAffine; end
struct CFold; kind::Int32; phase::Int32; body::Int32; weight::Int32; scan::Int32; reserved::Int32; end
struct COutput; value::Int32; term::Int32; full::Int32; accumulate::Int32; index::CAffine; end
struct FloorDesc
    kind::Int32; rank::Int32; extents::NTuple{4, Int64}; reduced::UInt32
    n_values::Int32; n_terms::Int32; n_folds::Int32; n_outputs::Int32; flags::Int32
    values::Ptr{FloorValue}; terms::Ptr{CTerm}; folds::Ptr{CFold}; outputs::Ptr{COutput}
end

const FLOOR_FN = IdDict{Any, Int32}(+ => 0, - => 1, * => 2, / => 3, abs => 5, abs2 => 6, sqrt => 7, exp => 8,
    log => 9, tanh => 10, sin => 11, cos => 12, log1p => 13, expm1 => 14, (^) => 15, max => 16, min => 17,
    (<) => 18, (<=) => 19, (>) => 20, (>=) => 21, (==) => 22, (!=) => 23, ifelse => 24, round => 25,
    floor => 26, ceil => 27, sign => 28, clamp => 29, fma => 30, inv => 31,
    Tempest.Compiler.IR.Cast{Tempest.BFloat16}() => 32)

# A fold value's (kind, observe): SumFold, MaxFold, MinFold, ProdFold; the
# exponential and square laws with their Statistic / Sum(1) / LOGSUMEXP observes.
function floor_fold(fold)
    F = Tempest.Compiler.IR
    fold isa F.SumFold && return (0, 0)
    fold isa F.ProdFold && return (1, 0)
    fold isa F.MaxFold && return (2, 0)
    fold isa F.MinFold && return (3, 0)
    if fold isa F.Relative
        kind = fold.law isa F.Exponential ? 4 : fold.law isa F.Square ? 5 : throw(ArgumentError("fold law"))
        obs = fold.observe isa F.Statistic ? 1 : fold.observe isa F.Sum ? 2 : kind == 4 ? 3 : throw(ArgumentError("observe"))
        return (kind, obs)
    end
    throw(ArgumentError("the generated floor has no fold $(typeof(fold))"))
end

# `gathered(atom)` adds the load an Indirect atom reads and returns its term number.
function caffine(e, gathered)
    IR = Tempest.Compiler.IR
    c = zeros(Int64, 4)
    gather, gc = Int32(-1), 0
    parts = CPart[]
    for (atom, k) in e.terms
        if atom isa IR.Var
            c[atom.n] += k
        elseif atom isa IR.Indirect && gather < 0
            gather, gc = gathered(atom), k
        elseif (atom isa IR.Div || atom isa IR.Mod) && length(parts) < 2
            inner = zeros(Int64, 4)
            for (a, j) in atom.e.terms
                a isa IR.Var || throw(ArgumentError("floor div / mod atoms take positions"))
                inner[a.n] += j
            end
            push!(parts, CPart(atom isa IR.Div ? 1 : 2, 0, atom.d, k, atom.e.constant, Tuple(inner)))
        else
            throw(ArgumentError("floor addresses take positions, two div / mod atoms and one gathered index"))
        end
    end
    while length(parts) < 2
        push!(parts, NO_PART)
    end
    CAffine(e.constant, Tuple(c), gather, 0, gc, (parts[1], parts[2]))
end

# The group as th_floor_desc arrays; `slots` numbers its values, `buffers` their storage.
function floor_descriptor(graph, g, slots, buffers)
    C = Tempest.Compiler
    terms, index = CTerm[], IdDict{Any, Int32}()
    folds = [r for r in g.reductions]
    fold_no = Dict(r => Int32(i - 1) for (i, r) in enumerate(folds))
    z = CAffine(0, (0, 0, 0, 0), -1, 0, 0, (NO_PART, NO_PART))
    # An Indirect atom reads value `a.value` at `a.index`: a load term of its own.
    gathered(a) = add!(C.IR.Load(a.value, a.index))
    function add!(t)
        haskey(index, t) && return index[t]
        ct = if t isa C.IR.Load
            CTerm(0, 0, (0, 0, 0), findfirst(==(t.value), slots) - 1, 0, 0f0,
                  caffine(C.address(graph.values[t.value], t.index, C.Domain(g.domain)), gathered))
        elseif t isa C.IR.Lit
            CTerm(1, 0, (0, 0, 0), 0, 0, Float32(t.value), z)
        elseif t isa C.IR.Ix
            CTerm(2, 0, (0, 0, 0), 0, 0, 0f0, caffine(t.expr, gathered))
        elseif t isa C.IR.Stat
            CTerm(3, 0, (0, 0, 0), fold_no[t.value], floor_fold(graph.values[t.value].definition.fold)[2], 0f0, z)
        elseif t isa C.IR.Apply
            a = Int32[add!(x) for x in t.args]
            CTerm(4, FLOOR_FN[t.f], (get(a, 1, 0), get(a, 2, 0), get(a, 3, 0)), 0, 0, 0f0, z)
        else
            throw(ArgumentError("the generated floor has no term $(typeof(t))"))
        end
        push!(terms, ct)
        index[t] = Int32(length(terms) - 1)
    end
    # A scan group's scans (Scan definitions, inclusive or exclusive) and its plain folds.
    scan_of(d) = d isa C.IR.Scan ? (d.exclusive ? 2 : 1) : 0
    cfolds = [CFold(floor_fold(graph.values[r].definition.fold)[1], g.phase[r], add!(g.terms[r]), -1,
                    scan_of(graph.values[r].definition), 0) for r in folds]
    outs = [COutput(findfirst(==(m), slots) - 1, add!(g.terms[m]), graph.values[m].dims == g.domain, 0,
                    caffine(C.address(graph.values[m], C.identity_index(g.domain), C.Domain(g.domain)), gathered))
            for m in g.outputs]
    code(T) = T === Float32 ? 0 : T === Tempest.BFloat16 ? 1 : T === Int32 ? 2 : T === Int64 ? 3 :
        throw(ArgumentError("the generated floor has no $T values"))
    vals = [FloorValue(code(graph.values[v].eltype), 0, C.storage_length(graph.values[v]),
                       address(buffers[i])) for (i, v) in enumerate(slots)]
    ext = ntuple(k -> k <= length(g.domain) ? Int64(g.domain[k]) : 1, 4)
    reduced = UInt32(sum((1 << (k - 1) for k in C.primary_axes(graph, g)); init = 0))
    (vals, terms, cfolds, outs, ext, reduced, floor_kind(g.kind))
end

# The group kinds the generated floor takes, by name; any other kind throws,
# so that the build falls back to its next option instead of dropping state.
function floor_kind(kind)
    C = Tempest.Compiler
    kind isa C.PointwiseKind && return Int32(0)
    kind isa C.ReductionKind && return Int32(1)
    kind isa C.ScanKind && return Int32(2)
    throw(ArgumentError("the generated floor takes pointwise, reduction and scan groups, not $(typeof(kind))"))
end

function build_floor(target::HIPTarget, p, g, buffers)
    slots = Tempest.Compiler.kernel_slots(p, g, Tempest.Compiler.floor_stored(p, g))
    vals, terms, folds, outs, ext, reduced, kind = floor_descriptor(p.graph, g, slots, [buffers[v] for v in slots])
    GC.@preserve vals terms folds outs begin
        reverse = kind == 2 && p.graph.values[first(g.reductions)].definition.reverse ? 1 : 0
        d = Ref(FloorDesc(kind, length(g.domain), ext, reduced,
                          length(vals), length(terms), length(folds), length(outs), reverse,
                          pointer(vals), pointer(terms), pointer(folds), pointer(outs)))
        out = Ref{Ptr{Cvoid}}()
        check(ccall((:th_build_floor, LIB), Cint, (Ptr{FloorDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_floor")
    end
    HIPLaunch(out[], Any[buffers[v] for v in slots])
end

end # module
