# HIPExt: Tempest's MI355X target over libtempest_hip, as a package extension.
#
# The Julia side a Tempest maintainer adds to put the HIP backend behind
# `compile`: a `HIPTarget` implementing the Target protocol
# (src/Compiler/runtime/target.jl), the floor for every group kind
# (`build_floor`, src/Compiler/runtime/runtime.jl:1319-1335), and libraries
# implementing the Implement interface (src/Compiler/Implement/library.jl):
# products (the templates of ext/cuBLASExt.jl:23-27), the products' fused
# epilogues, attention in cuDNN's form (ext/cuDNNExt.jl:29-51) with its
# backward, the fused row programs and the chunked gated DeltaNet.  Every
# device operation is a `ccall` into libtempest_hip (include/tempest_hip.h); a
# non-zero status becomes an exception, which the cover catches to fall back
# to its next option (src/Compiler/cover/choose.jl:1014-1025).
#
# No Julia toolchain exists where this backend was built, so this file has not
# been run; tests/test_julia_binding.py checks every `ccall` against the
# header (symbol, argument count, C types), every struct mirror against gcc's
# layout of the header's struct, every method that extends one of Tempest's
# functions against the reference's methods of it (no ambiguity, not shadowed),
# the Target protocol against what CUDATarget specialises, and the calls the
# runtime makes on a slot's storage against the methods here; the same calls,
# argument for argument, are exercised by the Python host in tempest.jl_amd/tempest_hip.
module HIPExt

using Tempest
import Tempest.Compiler: allocate, upload, upload!, download!, bindable, pointable, capture, recapture, retarget!,
    replay, release, device_name, toolchain, measurable, time_launch, device_rates, quiesce, build_floor,
    implementations, numerics, permits_rewrites, rounded_backward, deterministic, product_class,
    target_for, device_of, default_device, on_device, task_stream
using Tempest.Compiler.Implement: Library, Template, Binding, Strided, Work
import Tempest.Compiler.Implement: templates, supports, build, estimate, repoints, repoint!, loaded, in_place, package_of

const C = Tempest.Compiler

const LIB = get(ENV, "TEMPEST_HIP_LIBRARY", joinpath(@__DIR__, "..", "libtempest_hip.so"))

function check(status::Cint, what)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:th_last_error, LIB), Cstring, ()))
    throw(ErrorException("$what failed ($status): $msg"))
end

# ---- device storage -----------------------------------------------------------------

"""
    HIPPool(device, reserve)

One reserved range of `reserve` bytes of device addresses (th_pool_create):
`planned` allocates a slot at a time (runtime.jl:415), and every slot of
every executable lands in that range.  Every buffer taken from it holds it;
the library releases the range when the pool is destroyed and its last block
is freed, in whichever order the collector finalizes them.
"""
mutable struct HIPPool
    handle::Ptr{Cvoid}
    device::Int
    function HIPPool(device::Integer, reserve::Integer)
        check(ccall((:th_init, LIB), Cint, (Cint,), device), "th_init")
        out = Ref{Ptr{Cvoid}}()
        check(ccall((:th_pool_create, LIB), Cint, (UInt64, Ptr{Ptr{Cvoid}}), reserve, out), "th_pool_create")
        finalizer(p -> ccall((:th_pool_destroy, LIB), Cint, (Ptr{Cvoid},), p.handle), new(out[], Int(device)))
    end
end

"""
    HIPBuffer{T}(pool, n)

`n` elements of `T` on the device, a block of `pool`: a dense vector whose
`pointer` is the device address, as `planned` makes a slot (`allocate`) and
views it (`slot_view(slot, T, n) = reinterpret(T, view(slot, 1:n*sizeof(T)))`,
runtime.jl:605).  Elements read and written one at a time are copied one at a
time; `copyto!` between device arrays, and between them and `Array`s, copies
in one piece.
"""
mutable struct HIPBuffer{T} <: DenseVector{T}
    ptr::Ptr{T}
    n::Int
    pool::HIPPool
    function HIPBuffer{T}(pool::HIPPool, n::Integer) where {T}
        isbitstype(T) && sizeof(T) > 0 || throw(ArgumentError("a device buffer holds bits types, not $T"))
        out = Ref{Ptr{Cvoid}}()
        check(ccall((:th_pool_alloc, LIB), Cint, (Ptr{Cvoid}, UInt64, UInt64, Ptr{Ptr{Cvoid}}),
            pool.handle, max(n, 1) * sizeof(T), 256, out), "th_pool_alloc")
        b = new{T}(Ptr{T}(out[]), Int(n), pool)
        finalizer(x -> ccall((:th_pool_free, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}), x.pool.handle, x.ptr), b)
    end
end

Base.size(b::HIPBuffer) = (b.n,)
Base.length(b::HIPBuffer) = b.n
Base.IndexStyle(::Type{<:HIPBuffer}) = IndexLinear()
Base.elsize(::Type{<:HIPBuffer{T}}) where {T} = sizeof(T)
Base.sizeof(b::HIPBuffer{T}) where {T} = b.n * sizeof(T)
Base.pointer(b::HIPBuffer) = b.ptr
Base.pointer(b::HIPBuffer{T}, i::Integer) where {T} = b.ptr + (i - 1) * sizeof(T)
Base.unsafe_convert(::Type{Ptr{T}}, b::HIPBuffer{T}) where {T} = b.ptr
Base.similar(b::HIPBuffer, ::Type{T}, dims::Dims) where {T} =
    length(dims) == 1 ? HIPBuffer{T}(b.pool, dims[1]) : reshape(HIPBuffer{T}(b.pool, prod(dims)), dims)

function Base.getindex(b::HIPBuffer{T}, i::Int) where {T}
    @boundscheck checkbounds(b, i)
    x = Ref{T}()
    check(ccall((:th_download, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t), x, pointer(b, i), sizeof(T)), "th_download")
    x[]
end

function Base.setindex!(b::HIPBuffer{T}, v, i::Int) where {T}
    @boundscheck checkbounds(b, i)
    x = Ref{T}(convert(T, v))
    check(ccall((:th_upload, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t), pointer(b, i), x, sizeof(T)), "th_upload")
    b
end

# The forms a slot's storage takes in Tempest's runtime, each contiguous on
# the device: a buffer, a range of one, a reinterpretation of either (a slot's
# value, runtime.jl:605), and any of those reshaped (a result, runtime.jl:524).
const HIPSub{T} = SubArray{T, 1, <:HIPBuffer, <:Tuple{AbstractUnitRange}, true}
const HIPSlot{T} = Union{HIPBuffer{T}, HIPSub{T}, Base.ReinterpretArray{T, 1, <:Any, <:Union{HIPBuffer, HIPSub}}}
const HIPDense{T} = Union{HIPSlot{T}, Base.ReshapedArray{T, <:Any, <:HIPSlot}}

Base.pointer(x::HIPSub{T}) where {T} = pointer(parent(x)) + (first(only(parentindices(x))) - 1) * sizeof(T)
Base.pointer(x::Base.ReinterpretArray{T, 1, <:Any, <:Union{HIPBuffer, HIPSub}}) where {T} = Ptr{T}(pointer(parent(x)))
Base.pointer(x::Base.ReshapedArray{T, <:Any, <:HIPSlot}) where {T} = Ptr{T}(pointer(parent(x)))

# The pool a device array's storage was taken from.
pool_of(b::HIPBuffer) = b.pool
pool_of(x::HIPDense) = pool_of(parent(x))

device_address(x) = Ptr{Cvoid}(pointer(x))
bytes_of(x) = length(x) * sizeof(eltype(x))

function device_copy!(to::Ptr{Cvoid}, from::Ptr{Cvoid}, bytes)
    check(ccall((:th_copy, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t), to, from, bytes), "th_copy")
end

# Element ranges checked as Base's copyto! checks them; the copies run on the
# library's stream, in order with its launches (th_copy, th_upload, th_download).
function copy_span(dest, doff, src, soff, n)
    n >= 0 || throw(ArgumentError("tried to copy n=$n elements, but n should be nonnegative"))
    n == 0 && return false
    checkbounds(dest, doff:(doff + n - 1))
    checkbounds(src, soff:(soff + n - 1))
    true
end

function Base.copyto!(dest::HIPDense{T}, doff::Integer, src::HIPDense{T}, soff::Integer, n::Integer) where {T}
    copy_span(dest, doff, src, soff, n) &&
        device_copy!(device_address(dest) + (doff - 1) * sizeof(T), device_address(src) + (soff - 1) * sizeof(T), n * sizeof(T))
    dest
end

function Base.copyto!(dest::Array{T}, doff::Integer, src::HIPDense{T}, soff::Integer, n::Integer) where {T}
    copy_span(dest, doff, src, soff, n) &&
        check(ccall((:th_download, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
            pointer(dest, doff), device_address(src) + (soff - 1) * sizeof(T), n * sizeof(T)), "th_download")
    dest
end

function Base.copyto!(dest::HIPDense{T}, doff::Integer, src::Array{T}, soff::Integer, n::Integer) where {T}
    copy_span(dest, doff, src, soff, n) &&
        check(ccall((:th_upload, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Csize_t),
            device_address(dest) + (doff - 1) * sizeof(T), pointer(src, soff), n * sizeof(T)), "th_upload")
    dest
end

function whole(dest, src)
    length(dest) >= length(src) || throw(BoundsError(dest, eachindex(src)))
    length(src)
end
Base.copyto!(dest::HIPDense{T}, src::HIPDense{T}) where {T} = copyto!(dest, 1, src, 1, whole(dest, src))
Base.copyto!(dest::Array{T}, src::HIPDense{T}) where {T} = copyto!(dest, 1, src, 1, whole(dest, src))
Base.copyto!(dest::HIPDense{T}, src::Array{T}) where {T} = copyto!(dest, 1, src, 1, whole(dest, src))

# ---- the target ---------------------------------------------------------------------

"""
    HIPTarget(implementations...; device = 0, reserve = 64 << 30, precision = :full, deterministic = false)

One MI355X.  Its slots come from one reserved range of `reserve` bytes of
device addresses (`HIPPool`).  `implementations` are the libraries it offers
the cover, tried in order beside the floor; by default all of this
extension's.

- `precision`: the numerics policy for products of Float32 factors (as
  CUDATarget's, target.jl:42-44): `:full` keeps them in Float32 on the fp32
  matrix cores; `:bf16x3` splits each factor into two BFloat16 parts,
  `x = hi + lo`, and sums three bf16 products in Float32
  (`A_hi B_hi + A_hi B_lo + A_lo B_hi`, about 16 of Float32's 24 significant
  bits), on matrix cores sixteen times faster: the MI355X counterpart of
  `:tf32x3`, which this device has no TF32 for.
- `deterministic = true` keeps every sum's rounding independent of the order
  blocks run in (target.jl:229-231): the floor's folds by key then add their
  elements one at a time in the order of the items instead of by atomics,
  the one place this backend's sums depend on that order; every other kernel
  here folds in a fixed order either way.  `false` is the reference's default
  (target.jl:31).
"""
mutable struct HIPTarget <: C.Target
    implementations::Tuple
    device::Int
    pool::HIPPool
    precision::Symbol
    deterministic::Bool
    # The one inner constructor, so that Julia makes no field-by-field ones
    # that a call with five implementations would reach.
    function HIPTarget(::Val{:fields}, implementations::Tuple, device::Int, pool::HIPPool, precision::Symbol,
                       deterministic::Bool)
        precision in (:full, :bf16x3) || throw(ArgumentError("precision must be :full or :bf16x3, got $precision"))
        new(implementations, device, pool, precision, deterministic)
    end
end

HIPTarget(implementations...; device::Integer = 0, reserve::Integer = 64 << 30, precision::Symbol = :full,
    deterministic::Bool = false) =
    HIPTarget(Val(:fields), isempty(implementations) ? default_implementations() : implementations, Int(device),
        HIPPool(device, reserve), precision, deterministic)

# A target over an existing pool: what `target_for` gives for its buffers.
HIPTarget(pool::HIPPool; precision::Symbol = :full, deterministic::Bool = false) =
    HIPTarget(Val(:fields), default_implementations(), pool.device, pool, precision, deterministic)

default_implementations() = (HIPProducts(), HIPEpilogues(), HIPAttention(), HIPRows(), HIPDeltaNet())

Base.show(io::IO, t::HIPTarget) = print(io, "HIPTarget(", join(map(repr, t.implementations), ", "), "; device = ", t.device,
    ", precision = :", t.precision, t.deterministic ? ", deterministic = true" : "", ")")

# The options the compiler reads (target.jl:79-83,216-231; cover/cost.jl:132).
implementations(t::HIPTarget) = t.implementations
numerics(t::HIPTarget) = Symbol(t.precision, t.deterministic ? "-deterministic" : "")
# The row kernels and attention fold exponentials online, as the rewrite does.
permits_rewrites(::HIPTarget) = true
# The attention backward reads the forward's output as it was rounded to bf16.
rounded_backward(::HIPTarget) = true
deterministic(t::HIPTarget) = t.deterministic
# Half-precision products run as themselves, Float32 ones in the target's precision.
product_class(t::HIPTarget, T) = T === Float16 || T === Tempest.BFloat16 ? nameof(T) : t.precision

# Arrays and devices (target.jl:94-124,129-175).  One device per process: the
# library drives the device its first `th_init` named.
target_for(x::HIPDense) = HIPTarget(pool_of(x))
device_of(x::HIPDense) = pool_of(x).device
device_of(t::HIPTarget) = t.device
default_device(t::HIPTarget) = t.device
function on_device(f, t::HIPTarget, device::Int)
    device == t.device || throw(ArgumentError("libtempest_hip drives device $(t.device), not $device"))
    f()
end

allocate(t::HIPTarget, T, n) = HIPBuffer{T}(t.pool, n)
upload(t::HIPTarget, x) = upload!(t, allocate(t, eltype(x), length(x)), x)
# An array on the host other than an `Array` goes through one (as CUDA's
# target does, ext/CUDAExt.jl:33-36).
upload!(::HIPTarget, buffer, x) = copyto!(buffer, x isa Union{Array, HIPDense} ? vec(x) : vec(Array(x)))
download!(::HIPTarget, x, buffer) =
    x isa Union{Array, HIPDense} ? copyto!(x, buffer) : copyto!(x, reshape(copyto!(Array{eltype(buffer)}(undef, length(buffer)), buffer), size(x)))
bindable(::HIPTarget, x) = x isa HIPDense
# Kernels assume at most 16-byte alignment of what they are built on (th_launch_repoint checks it).
pointable(::HIPTarget, x, at) = x isa HIPDense && at % 16 == 0
quiesce(::HIPTarget) = check(ccall((:th_quiesce, LIB), Cint, ()), "th_quiesce")
# Every launch, copy and replay of the library goes to one stream: a task's
# stream is that one (ext/CUDAExt.jl:331-345 keeps CUDA's task streams).
function task_stream(::HIPTarget)
    s = Ref{Ptr{Cvoid}}()
    check(ccall((:th_get_stream, LIB), Cint, (Ptr{Ptr{Cvoid}},), s), "th_get_stream")
    s[]
end
quiesce(t::HIPTarget, ::Ptr{Cvoid}) = quiesce(t)

# ---- launches -----------------------------------------------------------------------

"""
One claim's launch: a th_launch*, the buffers it reads (kept alive), and
where each program value sits among its values: `(value, launch value,
element offset, element type)`, so that `repoint!` by a program value moves
every operand of it (ext/cuBLASExt.jl:270-276 keeps its operands so too).
"""
mutable struct HIPLaunch
    handle::Ptr{Cvoid}
    buffers::Vector{Any}
    operands::Vector{Tuple{Int, Int, Int, DataType}}
    function HIPLaunch(h, buffers, operands = Tuple{Int, Int, Int, DataType}[], pool::Union{Nothing, HIPPool} = nothing)
        l = new(h, buffers, operands)
        finalizer(x -> ccall((:th_launch_destroy, LIB), Cint, (Ptr{Cvoid},), x.handle), l)
        # Its workspace (partial sums, stored dS', ...) from the target's pool,
        # beside the slots, as the reference's floor takes its workspaces from
        # the target (runtime.jl:1326-1327); without a pool, allocated at the first run.
        if pool !== nothing
            n = Ref{UInt64}(0)
            check(ccall((:th_launch_workspace, LIB), Cint, (Ptr{Cvoid}, Ptr{UInt64}), h, n), "th_launch_workspace")
            if n[] > 0
                ws = HIPBuffer{UInt8}(pool, n[])
                check(ccall((:th_launch_set_workspace, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}), h, pointer(ws)),
                      "th_launch_set_workspace")
                push!(l.buffers, ws)
            end
        end
        l
    end
end
(l::HIPLaunch)() = check(ccall((:th_launch_run, LIB), Cint, (Ptr{Cvoid},), l.handle), "th_launch_run")
repoints(::HIPLaunch) = true
# `buffer` is any storage the runtime hands over: a buffer, a slot's view of
# one, the caller's array (runtime.jl:1091-1092,1130-1131).
function repoint!(l::HIPLaunch, value, buffer)
    for (v, i, offset, T) in l.operands
        v == value || continue
        check(ccall((:th_launch_repoint, LIB), Cint, (Ptr{Cvoid}, Cint, Ptr{Cvoid}), l.handle, i,
            device_address(buffer) + offset * sizeof(T)), "th_launch_repoint")
    end
    l
end

# The launch's operands from the Strided arrays it was built on, by its value numbers.
operands_of(pairs) = Tuple{Int, Int, Int, DataType}[(s.value, i, s.offset, s.eltype) for (i, s) in pairs if s !== nothing]

"""
The floor's launches for a group, run in order: the group's own kernel, or a
fold by key's start and elements (`keyed_kernels`, codegen/scalar.jl:496-522).
"""
struct HIPFloorRun
    launches::Vector{HIPLaunch}
end
(r::HIPFloorRun)() = foreach(l -> l(), r.launches)
repoints(::HIPFloorRun) = true
repoint!(r::HIPFloorRun, value, buffer) = (foreach(l -> repoint!(l, value, buffer), r.launches); r)

# ---- graphs -------------------------------------------------------------------------

"""
The copy a `Copy` step makes (runtime.jl:47-64), as a launch a graph records:
`length(c.to)` elements from `c.from` after its first `c.offset`.  Pointed
again at wherever the step's buffers are now, after the runtime repoints the
step (`point_copy!`).
"""
function copy_launch(c::C.Copy)
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_copy, LIB), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, UInt64, Ptr{Ptr{Cvoid}}),
        device_address(c.to), device_address(c.from) + c.offset * sizeof(eltype(c.from)), bytes_of(c.to), out), "th_build_copy")
    HIPLaunch(out[], Any[c.to, c.from])
end

function point_copy!(l::HIPLaunch, c::C.Copy)
    check(ccall((:th_launch_repoint, LIB), Cint, (Ptr{Cvoid}, Cint, Ptr{Cvoid}), l.handle, 0, device_address(c.to)),
        "th_launch_repoint")
    check(ccall((:th_launch_repoint, LIB), Cint, (Ptr{Cvoid}, Cint, Ptr{Cvoid}), l.handle, 1,
        device_address(c.from) + c.offset * sizeof(eltype(c.from))), "th_launch_repoint")
    l.buffers = Any[c.to, c.from]
    l
end

# The launches a step's run records as graph nodes, in order; nothing for a
# run this target cannot record (a recurrence stepped, runtime/stepped.jl),
# whose capture then replays the runs themselves.
recorded(run::HIPLaunch) = HIPLaunch[run]
recorded(run::HIPFloorRun) = run.launches
recorded(run::C.Copy) = bytes_of(run.to) > 0 ? HIPLaunch[copy_launch(run)] : HIPLaunch[]
recorded(run) = nothing

"""
A captured run of steps: a th_graph*, each step's run as captured, its
launches in the graph and where they start among the graph's (th_graph_retarget
numbers launches from 0, in capture order), and what the graph keeps alive.
"""
mutable struct HIPGraph
    handle::Ptr{Cvoid}
    runs::Vector{Any}
    launches::Vector{Vector{HIPLaunch}}
    first::Vector{Int}
    keep::Any
end

"""
Steps that replay faster launched one by one than as one graph, or that this
target cannot record: the steps' runs themselves, in order, each reading
where its launches read (as the reference's target records a run of
crossings, ext/CUDAExt.jl:561-566).
"""
struct HIPDirect
    runs::Vector{Any}
    keep::Any
end

# Whether `kernels` kernels replay faster as one graph than launched directly,
# from the costs th_dispatch_costs measures on this device once per process.
function graph_pays(kernels)
    base, gap, direct = Ref{Cdouble}(), Ref{Cdouble}(), Ref{Cdouble}()
    check(ccall((:th_dispatch_costs, LIB), Cint, (Ptr{Cdouble}, Ptr{Cdouble}, Ptr{Cdouble}), base, gap, direct),
        "th_dispatch_costs")
    base[] + kernels * gap[] < kernels * direct[]
end

# `steps` are `Scheduled` steps of one stream (schedule.jl:120-126): on one
# device their waits and signals order nothing beyond the stream's own order.
function capture(::HIPTarget, steps, keep)
    runs = Any[s.step.run for s in steps]
    launches = map(recorded, runs)
    any(isnothing, launches) && return HIPDirect(runs, keep)
    all_launches = reduce(vcat, launches; init = HIPLaunch[])
    graph_pays(sum(l -> launch_work(l).kernels, all_launches; init = 0)) || return HIPDirect(runs, keep)
    handles = Ptr{Cvoid}[l.handle for l in all_launches]
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_graph_capture, LIB), Cint, (Ptr{Ptr{Cvoid}}, Cint, Ptr{Ptr{Cvoid}}), handles, length(handles), out),
        "th_graph_capture")
    first = cumsum([0; length.(launches)])[1:end - 1]
    HIPGraph(out[], runs, launches, first, keep)
end
recapture(t::HIPTarget, g::Union{HIPGraph, HIPDirect}, steps, keep) = (release(t, g); capture(t, steps, keep))
replay(::HIPTarget, g::HIPGraph) = check(ccall((:th_graph_replay, LIB), Cint, (Ptr{Cvoid},), g.handle), "th_graph_replay")
replay(::HIPTarget, d::HIPDirect) = foreach(run -> run(), d.runs)
release(::HIPTarget, g::HIPGraph) =
    (g.handle == C_NULL || ccall((:th_graph_release, LIB), Cint, (Ptr{Cvoid},), g.handle); g.handle = C_NULL; nothing)
release(::HIPTarget, ::HIPDirect) = nothing

# `steps` are the moved steps' positions among those `capture` took
# (runtime.jl:1127: `[last(r.at[j]) for j in at]`).  Our kernels' argument
# layouts are known: the launches are repointed, then exactly their graph
# nodes take their arguments in place; nothing is learned or re-recorded
# (ext/CUDAExt.jl:614-668 learns them).  A recording of the runs reads where
# its runs read: true (target.jl:526-528).
retarget!(::HIPTarget, ::HIPDirect, steps, moves, repoint) = (repoint(); true)
function retarget!(::HIPTarget, g::HIPGraph, steps, moves, repoint)
    repoint()
    for s in steps
        run = g.runs[s]
        run isa C.Copy && foreach(l -> point_copy!(l, run), g.launches[s])
        for j in 0:(length(g.launches[s]) - 1)
            check(ccall((:th_graph_retarget, LIB), Cint, (Ptr{Cvoid}, Cint), g.handle, g.first[s] + j), "th_graph_retarget")
        end
    end
    true
end

# ---- measuring ----------------------------------------------------------------------

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
time_launch(t::HIPTarget, r::HIPFloorRun) = sum(l -> time_launch(t, l), r.launches)

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

struct CWork
    bytes::Cdouble
    flops::Cdouble
    blocks::Int64
    kernels::Int32
    values::Int32
end

"A launch's algorithmic work as th_launch_work states it."
function launch_work(l::HIPLaunch)
    w = Ref{CWork}()
    check(ccall((:th_launch_work, LIB), Cint, (Ptr{Cvoid}, Ptr{CWork}), l.handle, w), "th_launch_work")
    w[]
end

function describe(l::HIPLaunch)
    buf = Vector{UInt8}(undef, 4096)
    check(ccall((:th_launch_describe, LIB), Cint, (Ptr{Cvoid}, Ptr{UInt8}, Csize_t), l.handle, buf, length(buf)),
        "th_launch_describe")
    unsafe_string(pointer(buf))
end

address(s::Strided) = device_address(s.buffer) + s.offset * sizeof(s.eltype)
address_or_null(s) = s === nothing ? C_NULL : address(s)

# ---- products (the templates of cuBLASProducts, ext/cuBLASExt.jl:23-36) ----------------

struct HIPProducts <: Library end
loaded(::Type{HIPProducts}) = true

product(A, B) = C.contract(A, B, (1, 3, 4), (3, 2, 4), (1, 2, 4))
widened(A, B) = product(Float32.(A), Float32.(B))
accumulated(A, B, D) = D .+ product(A, B)

const PRODUCTS = (Template(product; inputs = (A = (:m, :k, :b), B = (:k, :n, :b)), outputs = (:C,)),
    Template(widened; inputs = (A = (:m, :k, :b), B = (:k, :n, :b)), outputs = (:C,)),
    Template(accumulated; inputs = (A = (:m, :k, :b), B = (:k, :n, :b), D = (:m, :n, :b)), outputs = (:C,)))
const WIDENED, ACCUMULATED = 2, 3
templates(::HIPProducts, ::HIPTarget) = PRODUCTS

struct GemmDesc
    m::Int32; n::Int32; k::Int32; c_dtype::Int32; epilogue::Int32; tile::Int32
    a::Ptr{Cvoid}; a_m::Int64; a_k::Int64
    b::Ptr{Cvoid}; b_k::Int64; b_n::Int64
    c::Ptr{Cvoid}; c_ld::Int64
    bias::Ptr{Cvoid}; aux::Ptr{Cvoid}; aux_ld::Int64; aux_out::Ptr{Cvoid}; row_sums::Ptr{Cvoid}; loss::Ptr{Cvoid}
    batch::Int32; flags::Int32
    a_batch::Int64; b_batch::Int64; c_batch::Int64
    d::Ptr{Cvoid}; d_ld::Int64; d_batch::Int64
    splits::Int32; reserved2::Int32
end

const TH_F32, TH_BF16, TH_F16 = Int32(0), Int32(1), Int32(4)
const GEMM_F32_FACTORS, GEMM_F16_FACTORS, GEMM_ACCUMULATE, GEMM_BF16X3 = Int32(1), Int32(2), Int32(4), Int32(8)
dtype_code(T) = T === Float32 ? TH_F32 : T === Tempest.BFloat16 ? TH_BF16 : T === Float16 ? TH_F16 :
    throw(ArgumentError("libtempest_hip has no $T arrays"))
factor_flags(T) = T === Float32 ? GEMM_F32_FACTORS : T === Float16 ? GEMM_F16_FACTORS : Int32(0)

# A binding as th_gemm_desc, or nothing: Float32, Float16 or BFloat16
# factors of one type, a result of theirs or Float32, the result column-major
# (unit stride along m), and for `accumulated` a matrix added laid out as the
# result.  Any other strides the library takes (the library chooses the
# kernel and its tile: the 256 x 256 or a middle tile where it can, the general
# kernel else).  With `buffers = false` the addresses are null (`supports` is
# asked without storage).  `precision = :bf16x3` runs Float32 factors with a
# Float32 result as split bf16 (TH_GEMM_BF16X3).
function gemm_desc(b::Binding; buffers = true, precision = :full)
    A, B, Cr = b.arrays.A, b.arrays.B, b.arrays.C
    T, R = A.eltype, Cr.eltype
    T in (Float32, Float16, Tempest.BFloat16) && B.eltype === T && (R === T || R === Float32) || return nothing
    b.template == WIDENED && T === Float32 && return nothing
    e = b.extents
    Cr.strides[1] == 1 && Cr.strides[2] >= max(e.m, 1) || return nothing
    accumulate = b.template == ACCUMULATED
    D = accumulate ? b.arrays.D : nothing
    accumulate && !(D.eltype === R && D.strides == Cr.strides) && return nothing
    p(s) = buffers ? address_or_null(s) : C_NULL
    x3 = precision === :bf16x3 && T === Float32 && R === Float32 ? GEMM_BF16X3 : Int32(0)
    GemmDesc(e.m, e.n, e.k, dtype_code(R), 0, 0, p(A), A.strides[1], A.strides[2], p(B), B.strides[1], B.strides[2],
        p(Cr), Cr.strides[2], C_NULL, C_NULL, 0, C_NULL, C_NULL, C_NULL,
        e.b, factor_flags(T) | (accumulate ? GEMM_ACCUMULATE : Int32(0)) | x3, A.strides[3], B.strides[3], Cr.strides[3],
        p(D), accumulate ? D.strides[2] : 0, accumulate ? D.strides[3] : 0, 0, 0)
end

supports(::HIPProducts, ::HIPTarget, b::Binding) = gemm_desc(b; buffers = false) !== nothing
# D + A B reads each element of D before it writes the result there.
in_place(::HIPProducts, b::Binding) = b.template == ACCUMULATED

estimate(::HIPProducts, b::Binding, target, g) =
    [Work(g.bytes; flops = 2.0 * b.extents.m * b.extents.n * b.extents.k * b.extents.b, factor = b.arrays.A.eltype)]

product_operands(b::Binding) =
    operands_of(((0, b.arrays.A), (1, b.arrays.B), (2, b.arrays.C), (8, get(b.arrays, :D, nothing))))

# The descriptor with th_gemm_tune's choice of tile and splits.
function with_choice(d::GemmDesc, tile::Int32, splits::Int32)
    names = fieldnames(GemmDesc)
    vals = Any[getfield(d, f) for f in names]
    vals[findfirst(==(:tile), names)] = tile
    vals[findfirst(==(:splits), names)] = splits
    GemmDesc(vals...)
end

# TEMPEST_HIP_TUNE=1: the product's tile and splits measured on the device as
# it is built (th_gemm_tune: every tile that takes it, then the splits of the
# best, as the reference's cover searches its product tiles,
# ext/cuTileExt/contract.jl:12-27); otherwise the library's choice.  A product
# added to a matrix in place is not measured (each run would add it again).
function build(::HIPProducts, t::HIPTarget, b::Binding, resources)
    d = Ref(gemm_desc(b; precision = t.precision))
    if get(ENV, "TEMPEST_HIP_TUNE", "") == "1" && b.template != ACCUMULATED
        tile, splits, secs = Ref{Int32}(0), Ref{Int32}(0), Ref{Float64}(0)
        check(ccall((:th_gemm_tune, LIB), Cint, (Ptr{GemmDesc}, Ptr{Int32}, Ptr{Int32}, Ptr{Float64}),
            d, tile, splits, secs), "th_gemm_tune")
        d[] = with_choice(d[], tile[], splits[])
    end
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_gemm, LIB), Cint, (Ptr{GemmDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_gemm")
    l = HIPLaunch(out[], Any[s.buffer for s in values(b.arrays)], product_operands(b), t.pool)
    (l, "HIP product $(b.extents.m)×$(b.extents.n) summing $(b.extents.k)" *
        (b.extents.b > 1 ? ", batch $(b.extents.b)" : "") * (b.template == ACCUMULATED ? ", added to a matrix" : "") *
        ": " * describe(l))
end

# Products alike but for where their operands start: one launch of them all
# (th_build_gemm_grouped); products added to matrices are built one by one.
supports(lib::HIPProducts, target::HIPTarget, bs::Vector{Binding}) =
    all(b -> supports(lib, target, b) && b.template != ACCUMULATED, bs)

function build(::HIPProducts, t::HIPTarget, bs::Vector{Binding}, resources)
    descs = [gemm_desc(b; precision = t.precision) for b in bs]
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_gemm_grouped, LIB), Cint, (Ptr{GemmDesc}, Cint, Ptr{Ptr{Cvoid}}), descs, length(descs), out),
        "th_build_gemm_grouped")
    # Product i's value v is value 9 (i - 1) + v of the grouped launch.
    ops = reduce(vcat, [[(v, 9 * (i - 1) + j, o, T) for (v, j, o, T) in product_operands(b)] for (i, b) in enumerate(bs)])
    l = HIPLaunch(out[], Any[s.buffer for b in bs for s in values(b.arrays)], ops, t.pool)
    (l, "$(length(bs)) HIP products, one launch: " * describe(l))
end

# ---- the products' fused epilogues (config 3's groups, one kernel each) ------------------

struct HIPEpilogues <: Library end
loaded(::Type{HIPEpilogues}) = true

gelu(x) = x / 2 * (1 + tanh(oftype(x, 0.7978846) * (x + oftype(x, 0.044715) * x * x * x)))
gelu_grad(x) = (t = tanh(oftype(x, 0.7978846) * (x + oftype(x, 0.044715) * x * x * x));
    (1 + t) / 2 + x / 2 * (1 - t * t) * oftype(x, 0.7978846) * (1 + 3 * oftype(x, 0.044715) * x * x))
matmul(A, B) = C.contract(A, B, (1, 3), (3, 2), (1, 2))
# Z = W x .+ b stored, and H = gelu.(Z) (the MLP's hidden layer).
gelu_layer(W, x, b) = (z = eltype(W).(matmul(W, x) .+ b); (z, eltype(W).(gelu.(Float32.(z)))))
# y = W h .+ b; loss = sum(abs2, y); dy = 2y; db = sum(dy; dims = 2).
square_loss(W, h, b) = (y = eltype(W).(matmul(W, h) .+ b); dy = eltype(W).(2 .* Float32.(y));
    (sum(abs2, Float32.(y)), dy, eltype(W).(sum(Float32.(dy); dims = 2))))
# dz = (W' dy) .* gelu'(Z); db = sum(dz; dims = 2).
gelu_backward(Wt, dy, Z) = (dz = eltype(Wt).(eltype(Wt).(matmul(Wt, dy)) .* gelu_grad.(Float32.(Z)));
    (dz, eltype(Wt).(sum(Float32.(dz); dims = 2))))

const EPILOGUES = (Template(gelu_layer; inputs = (W = (:m, :k), x = (:k, :n), b = (:m,)), outputs = (:Z, :H)),
    Template(square_loss; inputs = (W = (:m, :k), x = (:k, :n), b = (:m,)), outputs = (:loss, :dy, :db)),
    Template(gelu_backward; inputs = (W = (:m, :k), x = (:k, :n), Z = (:m, :n)), outputs = (:dz, :db)))
templates(::HIPEpilogues, ::HIPTarget) = EPILOGUES

function epilogue_desc(b::Binding; buffers = true)
    W, X = b.arrays.W, b.arrays.x
    all(s -> s.eltype === Tempest.BFloat16, (W, X)) || return nothing
    e = b.extents
    all(n -> n % 8 == 0, (e.m, e.n, e.k)) && (1 in W.strides[1:2]) && (1 in X.strides[1:2]) || return nothing
    p(s) = buffers ? address_or_null(s) : C_NULL
    a = b.arrays
    if b.template == 1
        GemmDesc(e.m, e.n, e.k, TH_BF16, 1, 0, p(W), W.strides[1], W.strides[2], p(X), X.strides[1], X.strides[2],
            p(a.Z), a.Z.strides[2], p(a.b), C_NULL, 0, p(a.H), C_NULL, C_NULL, 1, 0, 0, 0, 0, C_NULL, 0, 0, 1, 0)
    elseif b.template == 2
        GemmDesc(e.m, e.n, e.k, TH_BF16, 2, 0, p(W), W.strides[1], W.strides[2], p(X), X.strides[1], X.strides[2],
            p(a.dy), a.dy.strides[2], p(a.b), C_NULL, 0, C_NULL, p(a.db), p(a.loss), 1, 0, 0, 0, 0, C_NULL, 0, 0, 1, 0)
    else
        GemmDesc(e.m, e.n, e.k, TH_BF16, 3, 0, p(W), W.strides[1], W.strides[2], p(X), X.strides[1], X.strides[2],
            p(a.dz), a.dz.strides[2], C_NULL, p(a.Z), a.Z.strides[2], C_NULL, p(a.db), C_NULL, 1, 0, 0, 0, 0, C_NULL,
            0, 0, 1, 0)
    end
end

supports(::HIPEpilogues, ::HIPTarget, b::Binding) = epilogue_desc(b; buffers = false) !== nothing

estimate(::HIPEpilogues, b::Binding, target, g) =
    [Work(g.bytes; flops = 2.0 * b.extents.m * b.extents.n * b.extents.k, factor = b.arrays.W.eltype)]

function build(::HIPEpilogues, t::HIPTarget, b::Binding, resources)
    d = Ref(epilogue_desc(b))
    out = Ref{Ptr{Cvoid}}()
    check(ccall((:th_build_gemm, LIB), Cint, (Ptr{GemmDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_gemm")
    a = b.arrays
    # Values: 0 a, 1 b, 2 c, 3 bias, 4 aux, 5 aux_out, 6 row_sums, 7 loss.
    named = b.template == 1 ? ((0, a.W), (1, a.x), (2, a.Z), (3, a.b), (5, a.H)) :
        b.template == 2 ? ((0, a.W), (1, a.x), (2, a.dy), (3, a.b), (6, a.db), (7, a.loss)) :
        ((0, a.W), (1, a.x), (2, a.dz), (4, a.Z), (6, a.db))
    l = HIPLaunch(out[], Any[s.buffer for s in values(a)], operands_of(named), t.pool)
    (l, ("GELU layer", "square loss", "GELU backward")[b.template] * " fused into a HIP product: " * describe(l))
end

# ---- attention (cuDNN's form, ext/cuDNNExt.jl:29-51, and its backward) ------------------

struct HIPAttention <: Library end
loaded(::Type{HIPAttention}) = true

# The labels of `contract`: features, query heads per key head, key heads,
# queries, batch, keys.
const D_, G_, H_, M_, B_, N_ = 1, 2, 3, 4, 5, 6

# Queries (features, query heads per key head, key heads, queries, batch):
# query head g + G h reads key head h, as libtempest_hip's grouped heads do.
function attention(q, k, v; causal, statistics = false)
    s = C.contract(Float32.(k), Float32.(q), (D_, H_, N_, B_), (D_, G_, H_, M_, B_), (N_, G_, H_, M_, B_)) .*
        Float32(inv(sqrt(size(q, 1))))
    causal && (s = ifelse.(reshape(1:size(s, 1), :, 1, 1, 1) .<= reshape(1:size(s, 4), 1, 1, 1, :), s, -Inf32))
    lse = Tempest.logsumexp(s; dims = 1)
    o = C.contract(v, exp.(s .- lse), (D_, H_, N_, B_), (N_, G_, H_, M_, B_), (D_, G_, H_, M_, B_))
    statistics ? (eltype(q).(o), lse) : eltype(q).(o)
end

# The gradient of sum(attention(q, k, v) .* dout) from the forward's o and
# lse (FlashAttention's formulas): P = exp(S - lse), dV = P' dO, dP = dO V',
# dS = P .* (dP .- rowsum(dO .* O)), dQ = dS K / sqrt(d), dK = dS' Q / sqrt(d).
function attention_backward(q, k, v, o, lse, dout; causal)
    scale = Float32(inv(sqrt(size(q, 1))))
    s = C.contract(Float32.(k), Float32.(q), (D_, H_, N_, B_), (D_, G_, H_, M_, B_), (N_, G_, H_, M_, B_)) .* scale
    causal && (s = ifelse.(reshape(1:size(s, 1), :, 1, 1, 1) .<= reshape(1:size(s, 4), 1, 1, 1, :), s, -Inf32))
    p = exp.(s .- lse)
    delta = sum(Float32.(dout) .* Float32.(o); dims = 1)
    dv = C.contract(p, Float32.(dout), (N_, G_, H_, M_, B_), (D_, G_, H_, M_, B_), (D_, H_, N_, B_))
    dp = C.contract(Float32.(v), Float32.(dout), (D_, H_, N_, B_), (D_, G_, H_, M_, B_), (N_, G_, H_, M_, B_))
    ds = p .* (dp .- reshape(delta, 1, size(delta)...))
    dq = C.contract(Float32.(k), ds, (D_, H_, N_, B_), (N_, G_, H_, M_, B_), (D_, G_, H_, M_, B_)) .* scale
    dk = C.contract(Float32.(q), ds, (D_, G_, H_, M_, B_), (N_, G_, H_, M_, B_), (D_, H_, N_, B_)) .* scale
    (eltype(q).(dq), eltype(k).(dk), eltype(v).(dv))
end

# Without and with the statistics, each without and with the causal mask (the
# `k`th is causal when `k` is even), then the backward, without and with it.
const ATTENTION = (Tuple(Template((q, k, v) -> attention(q, k, v; causal, statistics);
        inputs = (q = (:d, :g, :h, :m, :b), k = (:d, :h, :n, :b), v = (:e, :h, :n, :b)), outputs = statistics ? (:o, :lse) : (:o,))
        for statistics in (false, true) for causal in (false, true))...,
    Tuple(Template((q, k, v, o, lse, dout) -> attention_backward(q, k, v, o, lse, dout; causal);
        inputs = (q = (:d, :g, :h, :m, :b), k = (:d, :h, :n, :b), v = (:e, :h, :n, :b), o = (:e, :g, :h, :m, :b),
            lse = (:g, :h, :m, :b), dout = (:e, :g, :h, :m, :b)), outputs = (:dq, :dk, :dv))
        for causal in (false, true))...)
causal(b::Binding) = iseven(b.template)
backward(b::Binding) = b.template > 4
templates(::HIPAttention, ::HIPTarget) = ATTENTION

struct AttentionDesc
    batch::Int32; heads::Int32; kv_heads::Int32; seq::Int32; head_dim::Int32
    causal::Int32; scale::Float32; flags::Int32
    q::Ptr{Cvoid}; k::Ptr{Cvoid}; v::Ptr{Cvoid}; o::Ptr{Cvoid}; lse::Ptr{Cvoid}
    dout::Ptr{Cvoid}; dq::Ptr{Cvoid}; dk::Ptr{Cvoid}; dv::Ptr{Cvoid}
    q_strides::NTuple{3, Int64}; k_strides::NTuple{3, Int64}
    kv_seq::Int32; reserved::Int32
    starts::Ptr{Cvoid}; lengths::Ptr{Cvoid}
end
const ATTN_F32 = Int32(2)

# The query-side arrays' head stride: the query heads of a group next to one
# another (sh = G sg), as libtempest_hip's head index g + G h reads them.
function head_stride(s::Strided)
    g, h = s.size[2], s.size[3]
    sg, sh = s.strides[2], s.strides[3]
    g == 1 ? sh : (h == 1 || sh == g * sg) ? sg : nothing
end

# A binding as th_attention_desc, or nothing: bf16 or fp32 arrays, as many
# value features as key features, up to 256, each feature axis contiguous,
# the lse Float32 laid out (heads, positions, batch) with heads contiguous.
function attention_desc(b::Binding; buffers = true)
    a, e = b.arrays, b.extents
    T = a.q.eltype
    T in (Tempest.BFloat16, Float32) && all(s -> s.eltype === T, (a.k, a.v)) || return nothing
    e.d == e.e && 1 <= e.d <= 256 || return nothing
    sq = head_stride(a.q)
    sq === nothing && return nothing
    all(s -> s.strides[1] == 1, (a.q, a.k, a.v)) || return nothing
    lse = get(a, :lse, nothing)
    lse === nothing || (lse.eltype === Float32 && lse.strides[1] == 1 && lse.strides[2] == e.g &&
                        lse.strides[3] == e.g * e.h && lse.strides[4] == e.g * e.h * e.m) || return nothing
    p(s) = buffers ? address_or_null(s) : C_NULL
    bw = backward(b)
    AttentionDesc(e.b, e.g * e.h, e.h, e.m, e.d, causal(b) ? 1 : 0, Float32(inv(sqrt(e.d))), T === Float32 ? ATTN_F32 : 0,
        p(a.q), p(a.k), p(a.v), p(get(a, :o, nothing)), p(lse), bw ? p(a.dout) : C_NULL,
        bw ? p(a.dq) : C_NULL, bw ? p(a.dk) : C_NULL, bw ? p(a.dv) : C_NULL,
        (sq, a.q.strides[4], a.q.strides[5]), (a.k.strides[2], a.k.strides[3], a.k.strides[4]), e.n, 0, C_NULL, C_NULL)
end

supports(::HIPAttention, ::HIPTarget, b::Binding) = attention_desc(b; buffers = false) !== nothing

function estimate(::HIPAttention, b::Binding, target, g)
    e = b.extents
    flops = 2.0 * (e.d + e.e) * e.g * e.h * e.m * e.b * e.n * (backward(b) ? 2.5 : 1.0)
    [Work(g.bytes; flops = causal(b) ? flops / 2 : flops, factor = b.arrays.q.eltype)]
end

function build(::HIPAttention, t::HIPTarget, b::Binding, resources)
    d = Ref(attention_desc(b))
    out = Ref{Ptr{Cvoid}}()
    a = b.arrays
    if backward(b)
        check(ccall((:th_build_attention_bwd, LIB), Cint, (Ptr{AttentionDesc}, Ptr{Ptr{Cvoid}}), d, out),
            "th_build_attention_bwd")
        named = ((0, a.q), (1, a.k), (2, a.v), (3, a.o), (4, a.lse), (5, a.dout), (6, a.dq), (7, a.dk), (8, a.dv))
    else
        check(ccall((:th_build_attention_fwd, LIB), Cint, (Ptr{AttentionDesc}, Ptr{Ptr{Cvoid}}), d, out),
            "th_build_attention_fwd")
        named = ((0, a.q), (1, a.k), (2, a.v), (3, a.o), (4, get(a, :lse, nothing)))
    end
    l = HIPLaunch(out[], Any[s.buffer for s in values(a)], operands_of(named), t.pool)
    (l, "HIP attention" * (backward(b) ? " backward" : "") * (causal(b) ? ", causal" : "") * ": " * describe(l))
end

# ---- the fused row programs (the cuTile resident sketch for these folds) -----------------

struct HIPRows <: Library end
loaded(::Type{HIPRows}) = true

softmax_fwd(x) = exp.(x .- Tempest.logsumexp(x; dims = 1))
layernorm_fwd(x) = (m = sum(x; dims = 1) ./ size(x, 1); v = sum(abs2, x .- m; dims = 1) ./ size(x, 1);
    (x .- m) ./ sqrt.(v .+ 1.0f-5))
softmax_grad(x, g) = (y = softmax_fwd(x); (sum(y .* g), y .* (g .- sum(y .* g; dims = 1))))
function layernorm_grad(x, g)
    n = size(x, 1)
    m = sum(x; dims = 1) ./ n
    v = sum(abs2, x .- m; dims = 1) ./ n
    r = 1 ./ sqrt.(v .+ 1.0f-5)
    y = (x .- m) .* r
    (sum(y .* g), r .* (g .- sum(g; dims = 1) ./ n .- y .* (sum(g .* y; dims = 1) ./ n)))
end
const ROWS = (Template(softmax_grad; inputs = (x = (:n, :r), g = (:n, :r)), outputs = (:loss, :dx)),
    Template(layernorm_grad; inputs = (x = (:n, :r), g = (:n, :r)), outputs = (:loss, :dx)),
    Template(softmax_fwd; inputs = (x = (:n, :r),), outputs = (:y,)),
    Template(layernorm_fwd; inputs = (x = (:n, :r),), outputs = (:y,)))
templates(::HIPRows, ::HIPTarget) = ROWS

# Float32 rows, contiguous, the output laid out as the input.
function supports(::HIPRows, ::HIPTarget, b::Binding)
    x = b.arrays.x
    out = b.template <= 2 ? b.arrays.dx : b.arrays.y
    x.eltype === Float32 && out.eltype === Float32 && x.strides[1] == 1 && out.strides == x.strides || return false
    b.template <= 2 ? b.arrays.g.strides == x.strides : b.extents.n <= 16384
end

function build(::HIPRows, t::HIPTarget, b::Binding, resources)
    a, e = b.arrays, b.extents
    out = Ref{Ptr{Cvoid}}()
    if b.template == 1
        check(ccall((:th_build_softmax_grad, LIB), Cint,
            (Int64, Int32, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Ptr{Cvoid}}),
            e.r, e.n, a.x.strides[2], address(a.x), address(a.g), address(a.dx), address(a.loss), out), "th_build_softmax_grad")
        named = ((0, a.x), (1, a.g), (2, a.dx), (3, a.loss))
    elseif b.template == 2
        check(ccall((:th_build_layernorm_grad, LIB), Cint,
            (Int64, Int32, Int64, Float32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Ptr{Cvoid}}),
            e.r, e.n, a.x.strides[2], 1.0f-5, address(a.x), address(a.g), address(a.dx), address(a.loss), out),
            "th_build_layernorm_grad")
        named = ((0, a.x), (1, a.g), (2, a.dx), (3, a.loss))
    elseif b.template == 3
        check(ccall((:th_build_softmax_fwd, LIB), Cint, (Int64, Int32, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Ptr{Cvoid}}),
            e.r, e.n, a.x.strides[2], address(a.x), address(a.y), out), "th_build_softmax_fwd")
        named = ((0, a.x), (1, a.y))
    else
        check(ccall((:th_build_layernorm_fwd, LIB), Cint, (Int64, Int32, Int64, Float32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Ptr{Cvoid}}),
            e.r, e.n, a.x.strides[2], 1.0f-5, address(a.x), address(a.y), out), "th_build_layernorm_fwd")
        named = ((0, a.x), (1, a.y))
    end
    l = HIPLaunch(out[], Any[s.buffer for s in values(a)], operands_of(named), t.pool)
    (l, ("softmax gradient", "LayerNorm gradient", "softmax", "LayerNorm")[b.template] * ", rows resident: " * describe(l))
end

# ---- the chunked gated DeltaNet (examples/deltanet.jl) ------------------------------------

struct HIPDeltaNet <: Library end
loaded(::Type{HIPDeltaNet}) = true

# The gated delta rule token by token (examples/deltanet.jl:89-101): per
# (head, batch), S = exp(a_t) (I - beta_t k_t k_t') S + beta_t k_t v_t' from
# zero, o_t = S' q_t; q, k, v (d, heads, positions, batch), a and beta
# (heads, positions, batch).
function deltanet(q, k, v, a, beta)
    d, H, T, B = size(q)
    o = similar(q)
    for b in 1:B, h in 1:H
        S = zeros(Float32, d, size(v, 1))
        for t in 1:T
            kt, vt, qt = Float32.(k[:, h, t, b]), Float32.(v[:, h, t, b]), Float32.(q[:, h, t, b])
            S = exp(a[h, t, b]) .* (S .- beta[h, t, b] .* kt * (kt' * S)) .+ beta[h, t, b] .* kt * vt'
            o[:, h, t, b] = eltype(q).(S' * qt)
        end
    end
    o
end
deltanet_grad(q, k, v, a, beta, dout) = Tempest.gradient((q, k, v, a, beta) -> sum(deltanet(q, k, v, a, beta) .* dout),
    q, k, v, a, beta)
const DELTANET = (Template(deltanet; inputs = (q = (:d, :h, :t, :b), k = (:d, :h, :t, :b), v = (:e, :h, :t, :b),
        a = (:h, :t, :b), beta = (:h, :t, :b)), outputs = (:o,)),
    Template(deltanet_grad; inputs = (q = (:d, :h, :t, :b), k = (:d, :h, :t, :b), v = (:e, :h, :t, :b),
        a = (:h, :t, :b), beta = (:h, :t, :b), dout = (:e, :h, :t, :b)), outputs = (:dq, :dk, :dv, :da, :dbeta)))
templates(::HIPDeltaNet, ::HIPTarget) = DELTANET

struct DeltaNetDesc
    batch::Int32; heads::Int32; seq::Int32; dk::Int32; dv::Int32; chunk::Int32
    q::Ptr{Cvoid}; k::Ptr{Cvoid}; v::Ptr{Cvoid}; a::Ptr{Cvoid}; beta::Ptr{Cvoid}
    o::Ptr{Cvoid}; dout::Ptr{Cvoid}; dq::Ptr{Cvoid}; dk_out::Ptr{Cvoid}; dv_out::Ptr{Cvoid}
    da::Ptr{Cvoid}; dbeta::Ptr{Cvoid}
    strides::NTuple{3, Int64}; gate_strides::NTuple{3, Int64}
end

function supports(::HIPDeltaNet, ::HIPTarget, b::Binding)
    a, e = b.arrays, b.extents
    e.d == 128 && e.e == 128 && e.t % 64 == 0 || return false
    all(s -> s.eltype === Tempest.BFloat16 && s.strides[1] == 1 && s.strides == a.q.strides, (a.q, a.k, a.v)) &&
        all(s -> s.eltype === Float32 && s.strides == a.a.strides, (a.a, a.beta))
end

# The chunked form's products (examples/deltanet.jl:58-86), chunk 64, d = 128:
# per chunk about 12.9 Mflop forward, three times that with the gradient.
function estimate(::HIPDeltaNet, b::Binding, target, g)
    e = b.extents
    chunks = e.h * e.b * (e.t ÷ 64)
    [Work(g.bytes; flops = chunks * 12.9e6 * (b.template == 2 ? 3.0 : 1.0), factor = Float32)]
end

function build(::HIPDeltaNet, t::HIPTarget, b::Binding, resources)
    a, e = b.arrays, b.extents
    grad = b.template == 2
    p(s) = address_or_null(s)
    d = Ref(DeltaNetDesc(e.b, e.h, e.t, 128, 128, 64, p(a.q), p(a.k), p(a.v), p(a.a), p(a.beta),
        grad ? C_NULL : p(a.o), grad ? p(a.dout) : C_NULL, grad ? p(a.dq) : C_NULL, grad ? p(a.dk) : C_NULL,
        grad ? p(a.dv) : C_NULL, grad ? p(a.da) : C_NULL, grad ? p(a.dbeta) : C_NULL,
        (a.q.strides[2], a.q.strides[3], a.q.strides[4]), (a.a.strides[1], a.a.strides[2], a.a.strides[3])))
    out = Ref{Ptr{Cvoid}}()
    name = grad ? :th_build_deltanet : :th_build_deltanet_fwd
    if grad
        # The gradient's launch computes o as well: a scratch of its own.
        check(ccall((:th_build_deltanet, LIB), Cint, (Ptr{DeltaNetDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_deltanet")
        named = ((0, a.q), (1, a.k), (2, a.v), (3, a.a), (4, a.beta), (6, a.dout), (7, a.dq), (8, a.dk), (9, a.dv),
            (10, a.da), (11, a.dbeta))
    else
        check(ccall((:th_build_deltanet_fwd, LIB), Cint, (Ptr{DeltaNetDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_deltanet_fwd")
        named = ((0, a.q), (1, a.k), (2, a.v), (3, a.a), (4, a.beta), (5, a.o))
    end
    l = HIPLaunch(out[], Any[s.buffer for s in values(a)], operands_of(named), t.pool)
    (l, "chunked gated DeltaNet" * (grad ? " gradient" : "") * ": " * describe(l))
end

# ---- the floor: any group, generated -----------------------------------------------------
#
# The reference's floor turns a group into Julia code (scalar_kernel,
# src/Compiler/codegen/scalar.jl:186-440) and CUDA compiles it (floor_launch,
# ext/CUDAExt.jl:926-937).  Here the group's terms cross the C ABI as arrays
# (th_floor_desc) and libtempest_hip writes and compiles the gfx950 kernel.
# Pointwise, reduction, scan and recurrence groups; Var atoms in addresses,
# up to two Div or Mod atoms of positions and one Indirect atom (a gathered
# index); Recomputed terms (not nested); the functions of FLOOR_FN; the folds
# of `floor_fold`; folds by key that add (SumFold) or write (Overwrite).  Any
# other form throws, and the build falls back to its next option.

struct FloorValue; dtype::Int32; reserved::Int32; length::Int64; ptr::Ptr{Cvoid}; end
struct CPart; kind::Int32; reserved::Int32; divisor::Int64; coeff::Int64; constant::Int64; inner::NTuple{4, Int64}; end
struct CAffine
    constant::Int64; coeff::NTuple{4, Int64}; gather::Int32; reserved::Int32; gather_coeff::Int64
    part::NTuple{2, CPart}
end
const NO_PART = CPart(0, 0, 1, 0, 0, (0, 0, 0, 0))
const NO_ADDRESS = CAffine(0, (0, 0, 0, 0), -1, 0, 0, (NO_PART, NO_PART))
struct CTerm; op::Int32; fn::Int32; args::NTuple{3, Int32}; ref::Int32; observe::Int32; lit::Float32; index::CAffine; end
struct CFold
    kind::Int32; phase::Int32; body::Int32; weight::Int32; scan::Int32; n_inner::Int32; inner::NTuple{4, Int64}
end
struct COutput; value::Int32; term::Int32; full::Int32; accumulate::Int32; index::CAffine; end
struct FloorDesc
    kind::Int32; rank::Int32; extents::NTuple{4, Int64}; reduced::UInt32
    n_values::Int32; n_terms::Int32; n_folds::Int32; n_outputs::Int32; flags::Int32
    values::Ptr{FloorValue}; terms::Ptr{CTerm}; folds::Ptr{CFold}; outputs::Ptr{COutput}
end

const GROUP_POINTWISE, GROUP_REDUCTION, GROUP_SCAN, GROUP_RECURRENCE = Int32(0), Int32(1), Int32(2), Int32(3)
const STEP_EACH, STEP_FIRST, STEP_LAST, STEP_CARRY = Int32(0), Int32(1), Int32(2), Int32(3)
const FLOOR_ORDERED = Int32(1 << 16)

const FLOOR_FN = IdDict{Any, Int32}(+ => 0, - => 1, * => 2, / => 3, abs => 5, abs2 => 6, sqrt => 7, exp => 8,
    log => 9, tanh => 10, sin => 11, cos => 12, log1p => 13, expm1 => 14, (^) => 15, max => 16, min => 17,
    (<) => 18, (<=) => 19, (>) => 20, (>=) => 21, (==) => 22, (!=) => 23, ifelse => 24, round => 25,
    floor => 26, ceil => 27, sign => 28, clamp => 29, fma => 30, inv => 31,
    Tempest.Compiler.IR.Cast{Tempest.BFloat16}() => 32)

# An extreme's combine (`Better{largest}`, program/tracing.jl:779-784).
better(f) = nameof(typeof(f)) === :Better ? typeof(f).parameters[1]::Bool : nothing

# A fold value's (kind, observe): SumFold, MaxFold, MinFold, ProdFold; the
# exponential and square laws with their Statistic / Sum(1) / LOGSUMEXP
# observes; findmax / findmin (a GenericFold combining by `Better`, its
# observe `first` the extreme, `last` its index).
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
    if fold isa F.GenericFold && better(fold.combine) !== nothing
        return (better(fold.combine) ? 7 : 8, fold.observe === last ? 1 : 0)
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

# A fold's element: a number, or (y, g) when the term is a tuple (a weighted
# element, a recurrence's pair, an extreme's element and index).
function element(t)
    IR = Tempest.Compiler.IR
    t isa IR.Apply && t.f === tuple && length(t.args) == 2 ? (t.args[1], t.args[2]) : (t, nothing)
end

"The group as th_floor_desc arrays; `slots` numbers its values, `buffers` their storage."
mutable struct FloorBuilder
    graph::Any
    g::Any
    slots::Vector{Int}
    domain::Tuple
    terms::Vector{CTerm}
    index::IdDict{Any, Int32}
    folds::Vector{CFold}
    fold_no::Dict{Int, Int32}
end

FloorBuilder(graph, g, slots, domain) = FloorBuilder(graph, g, slots, Tuple(domain), CTerm[], IdDict{Any, Int32}(), CFold[],
    Dict{Int, Int32}())

slot(b::FloorBuilder, v) = Int32(findfirst(==(v), b.slots) - 1)

function add!(b::FloorBuilder, t)
    haskey(b.index, t) && return b.index[t]
    IR, C_ = Tempest.Compiler.IR, Tempest.Compiler
    gathered(a) = add!(b, IR.Load(a.value, a.index))
    ct = if t isa IR.Load
        CTerm(0, 0, (0, 0, 0), slot(b, t.value), 0, 0f0,
              caffine(C_.address(b.graph.values[t.value], t.index, C_.Domain(b.domain)), gathered))
    elseif t isa IR.Lit
        CTerm(1, 0, (0, 0, 0), 0, 0, Float32(t.value), NO_ADDRESS)
    elseif t isa IR.Ix
        CTerm(2, 0, (0, 0, 0), 0, 0, 0f0, caffine(t.expr, gathered))
    elseif t isa IR.Stat
        CTerm(3, 0, (0, 0, 0), b.fold_no[t.value], floor_fold(b.graph.values[t.value].definition.fold)[2], 0f0, NO_ADDRESS)
    elseif t isa IR.Recomputed
        # A fold computed where it is read, over axes numbered after the domain's.
        length(b.domain) + length(t.extents) <= 4 || throw(ArgumentError("a recomputed fold's axes past four"))
        kind, obs = floor_fold(b.graph.values[t.value].definition.fold)
        y, w = element(t.body)
        f = CFold(kind, 0, add!(b, y), w === nothing ? -1 : add!(b, w), 0, length(t.extents),
            ntuple(k -> k <= length(t.extents) ? Int64(t.extents[k]) : 0, 4))
        push!(b.folds, f)
        CTerm(5, 0, (0, 0, 0), Int32(length(b.folds) - 1), obs, 0f0, NO_ADDRESS)
    elseif t isa IR.Apply
        a = Int32[add!(b, x) for x in t.args]
        CTerm(4, FLOOR_FN[t.f], (get(a, 1, 0), get(a, 2, 0), get(a, 3, 0)), 0, 0, 0f0, NO_ADDRESS)
    else
        throw(ArgumentError("the generated floor has no term $(typeof(t))"))
    end
    push!(b.terms, ct)
    b.index[t] = Int32(length(b.terms) - 1)
end

value_code(T) = T === Float32 ? 0 : T === Tempest.BFloat16 ? 1 : T === Int32 ? 2 : T === Int64 ? 3 :
    throw(ArgumentError("the generated floor has no $T values"))

function floor_values(b::FloorBuilder, buffers)
    C_ = Tempest.Compiler
    [FloorValue(value_code(b.graph.values[v].eltype), 0, C_.storage_length(b.graph.values[v]),
                device_address(buffers[i])) for (i, v) in enumerate(b.slots)]
end

function floor_desc(kind, domain, reduced, flags, vals, terms, folds, outs)
    ext = ntuple(k -> k <= length(domain) ? Int64(domain[k]) : 1, 4)
    FloorDesc(kind, length(domain), ext, reduced, length(vals), length(terms), length(folds), length(outs), flags,
              pointer(vals), pointer(terms), isempty(folds) ? C_NULL : pointer(folds), pointer(outs))
end

function floor_launch(kind, domain, reduced, flags, vals, terms, folds, outs, keep, operands, pool = nothing)
    out = Ref{Ptr{Cvoid}}()
    GC.@preserve vals terms folds outs begin
        d = Ref(floor_desc(kind, domain, reduced, flags, vals, terms, folds, outs))
        check(ccall((:th_build_floor, LIB), Cint, (Ptr{FloorDesc}, Ptr{Ptr{Cvoid}}), d, out), "th_build_floor")
    end
    HIPLaunch(out[], keep, operands, pool)
end

# The group's kinds by name; any other throws, so that the build falls back.
function floor_kind(kind)
    C_ = Tempest.Compiler
    kind isa C_.PointwiseKind && return GROUP_POINTWISE
    kind isa C_.ReductionKind && return GROUP_REDUCTION
    kind isa C_.ScanKind && return GROUP_SCAN
    kind isa C_.RecurrenceKind && return GROUP_RECURRENCE
    throw(ArgumentError("the generated floor takes pointwise, reduction, scan and recurrence groups, not $(typeof(kind))"))
end

mentions(a::CAffine, k) = a.coeff[k] != 0 || any(p -> p.kind != 0 && p.coeff != 0 && p.inner[k] != 0, a.part)

# A recurrence group's outputs (recurrence_kernel, codegen/scalar.jl:402-440):
# each member at its place, a state only at the first step, a member along
# none of the steps only at the last; a value carried into its state stored
# also one step on, at every step but the last.
function recurrence_outputs(b::FloorBuilder, gathered)
    C_ = Tempest.Compiler
    graph, g = b.graph, b.g
    (; axis, parallel) = C_.recurrence_axes(graph, g)
    states = C_.recurrence_states(graph, g.outputs)
    state_of = Dict(C_.carried_from(graph, c) => c for c in states)
    places = C_.recurrence_places(graph, g.outputs).places
    reverse = graph.values[first(states)].definition.reverse
    step = reverse ? -1 : 1
    domain = C_.Domain(b.domain)
    outs = COutput[]
    for m in g.outputs
        term = add!(b, g.terms[m])
        at = caffine(C_.address(graph.values[m], places[m], domain), gathered)
        once = !any(e -> C_.mentions(e, axis), places[m])
        rule = m in states ? STEP_FIRST : once ? STEP_LAST : STEP_EACH
        push!(outs, COutput(slot(b, m), term, rule, 0, at))
        if haskey(state_of, m)
            c = state_of[m]
            next = Base.setindex(places[m], C_.add(C_.var(axis), step, domain), axis)
            push!(outs, COutput(slot(b, c), term, STEP_CARRY, 0, caffine(C_.address(graph.values[c], next, domain), gathered)))
        end
    end
    reduced = UInt32(sum((1 << (k - 1) for k in eachindex(b.domain) if !(k in parallel)); init = 0))
    flags = Int32((reverse ? 1 : 0) | ((axis - 1) << 8))
    (outs, reduced, flags)
end

# A fold by key's two launches (keyed_kernels, codegen/scalar.jl:496-522):
# its storage set to the contents it starts from or the fold's initial state
# (unless `held` already), then each element added (SumFold, by atomics) or
# written (Overwrite) at the position its key names.  `ordered`, for a
# deterministic target, takes the elements one after another in the items'
# order (TH_FLOOR_ORDERED): no atomics, every run rounds alike.
function keyed_launches(graph, g, r, held, slots, buffers, operands, ordered, pool)
    C_, IR = Tempest.Compiler, Tempest.Compiler.IR
    val = graph.values[r]
    d = val.definition
    fold = d.fold
    (fold isa IR.SumFold || fold isa IR.Overwrite) || throw(ArgumentError("the floor folds by key by adding or writing"))
    launches = HIPLaunch[]
    keep = Any[buffers...]
    if !held
        b0 = FloorBuilder(graph, g, slots, val.dims)
        gathered0(a) = add!(b0, IR.Load(a.value, a.index))
        start = d.into === nothing ? add!(b0, IR.Lit(0.0f0)) : add!(b0, C_.stored_term(d.into))
        outs = [COutput(slot(b0, r), start, 1, 0, caffine(C_.address(val, C_.identity_index(val.dims), C_.Domain(val.dims)), gathered0))]
        push!(launches, floor_launch(GROUP_POINTWISE, val.dims, UInt32(0), Int32(0), floor_values(b0, buffers), b0.terms,
                                     b0.folds, outs, keep, operands, pool))
    end
    b = FloorBuilder(graph, g, slots, g.domain)
    gathered(a) = add!(b, IR.Load(a.value, a.index))
    t = add!(b, C_.stored_statistics(g.terms[r], graph, g))
    at = caffine(C_.address(val, C_.placement(graph, g, r), C_.Domain(g.domain)), gathered)
    outs = [COutput(slot(b, r), t, 1, fold isa IR.SumFold ? 1 : 0, at)]
    push!(launches, floor_launch(GROUP_POINTWISE, g.domain, UInt32(0), ordered ? FLOOR_ORDERED : Int32(0),
                                 floor_values(b, buffers), b.terms, b.folds, outs, keep, operands, pool))
    launches
end

# The floor for a group on this target, in place of the generic one
# (runtime.jl:1323-1335), whose kernels are Julia functions: the group's
# terms go to the library, which writes and compiles the kernel.  What the
# floor stores that the plan does not is kept in storage of its own, taken
# from the target's pool and held by the run, as the generic floor keeps it.
function build_floor(target::HIPTarget, p::C.Plan, g::C.Group, buffers)
    C_, IR = Tempest.Compiler, Tempest.Compiler.IR
    graph = p.graph
    stored = C_.floor_stored(p, g)
    slots = C_.kernel_slots(p, g, stored)
    own = Any[]
    function buffer(v)
        (buffers[v] !== nothing || p.stored[v]) && return buffers[v]
        b = allocate(target, graph.values[v].eltype, C_.storage_length(graph.values[v]))
        push!(own, b)
        b
    end
    bufs = Any[buffer(v) for v in slots]
    operands = Tuple{Int, Int, Int, DataType}[(v, i - 1, 0, UInt8) for (i, v) in enumerate(slots)]
    launches = HIPLaunch[]
    keyed = filter(r -> C_.keyed(graph, r), g.reductions)
    for r in keyed
        append!(launches, keyed_launches(graph, g, r, C_.starts_in_place(graph, r, buffers), slots, bufs, operands,
                                         deterministic(target), target.pool))
    end
    folds_in_place = [r for r in g.reductions if !(r in keyed)]
    if !isempty(folds_in_place) || g.kind isa C_.PointwiseKind || g.kind isa C_.RecurrenceKind
        b = FloorBuilder(graph, g, slots, g.domain)
        gathered(a) = add!(b, IR.Load(a.value, a.index))
        kind = floor_kind(g.kind)
        scan_of(d) = d isa IR.Scan ? (d.exclusive ? 2 : 1) : 0
        for (i, r) in enumerate(folds_in_place)
            b.fold_no[r] = Int32(i - 1)
        end
        # The folds run in phases come first; recomputed ones follow as their terms meet them.
        phased = CFold[]
        for r in folds_in_place
            y, w = element(g.terms[r])
            push!(phased, CFold(floor_fold(graph.values[r].definition.fold)[1], g.phase[r], add!(b, y),
                                w === nothing ? -1 : add!(b, w), scan_of(graph.values[r].definition), 0, (0, 0, 0, 0)))
        end
        if kind == GROUP_RECURRENCE
            outs, reduced, flags = recurrence_outputs(b, gathered)
        else
            outs = [COutput(slot(b, m), add!(b, g.terms[m]), graph.values[m].dims == g.domain, 0,
                            caffine(C_.address(graph.values[m], C_.identity_index(g.domain), C_.Domain(g.domain)), gathered))
                    for m in g.outputs if !(m in keyed)]
            reduced = UInt32(sum((1 << (k - 1) for k in C_.primary_axes(graph, g)); init = 0))
            reverse = kind == GROUP_SCAN && graph.values[first(folds_in_place)].definition.reverse
            flags = Int32(reverse ? 1 : 0)
        end
        # Recomputed folds were appended while the terms were added: renumber
        # their references after the phased folds.
        recomputed = b.folds
        folds = [phased; recomputed]
        terms = [t.op == 5 ? CTerm(t.op, t.fn, t.args, t.ref + length(phased), t.observe, t.lit, t.index) : t for t in b.terms]
        push!(launches, floor_launch(kind, g.domain, reduced, flags, floor_values(b, bufs), terms, folds, outs, Any[bufs...],
                                     operands, target.pool))
    end
    foreach(l -> append!(l.buffers, own), launches)
    run = HIPFloorRun(launches)
    (run, "HIP floor: " * join(map(describe, launches), "; "))
end

# The package the rates file keeps these libraries' lines under
# (tempest.jl_amd/rates/AMD_Instinct_MI355X.cold.rates.tsv: `HIP ...`), as
# Tempest's own libraries name theirs (Implement/packages.jl:42-44); by
# default it would be this module's name.
const HIPLibrary = Union{HIPProducts, HIPEpilogues, HIPAttention, HIPRows, HIPDeltaNet}
package_of(::HIPLibrary) = :HIP

end # module
