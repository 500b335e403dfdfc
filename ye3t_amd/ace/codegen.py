"""Generate a specialised HIP kernel for one :class:`ProductPlan` (stage 2 fast path).

The generic product kernel interprets the plan from LDS; this generator emits
the same DAG as straight-line code instead: every node value is a register,
every CG / symmetric-block coefficient an instruction literal, so a lane does
only the FMAs of its sample.  The source is compiled at run time (hipRTC, by
``ye3t_hip_product_plan_create_generated``) and cached per plan.

Kernel shape: ``grid = (ceil(samples / 64), chunk_count)``, 64 threads; lane =
sample.  Single-chunk plans stage the whole ``[64, F]`` output tile in LDS
(row stride ``F`` padded to odd, bank-conflict free both ways) and write it as
one contiguous block -- the tile's rows are consecutive in ``B`` -- with 16-byte
stores, so every output cache line is written whole by one wave.  Multi-chunk
plans own contiguous column ranges and flush ``GROUP`` columns at a time.
"""

import hashlib

from ye3t_amd.ace.program import _closure

GROUP = 32  # output columns staged per flush
CHAINS = 4  # independent partial sums per output component (persistent kernel)
STORE_BATCH = 16  # staged elements read from LDS ahead of their stores (generated parts)


def _ctype(dtype):
    return "double" if dtype == "f64" else "float"


def _check_in_dtype(dtype, in_dtype):
    """Density storage type of a kernel whose arithmetic is ``dtype``."""
    in_dtype = in_dtype or dtype
    if in_dtype not in ("f32", "f64") or (dtype == "f32" and in_dtype == "f64"):
        raise ValueError(f"unsupported density dtype {in_dtype!r} for {dtype} arithmetic")
    return in_dtype


def _lit(value, dtype):
    if dtype == "f64":
        return repr(float(value))
    return repr(float(value)) + "f"


def _chunks(plan, max_live, align=1):
    """``[(first, last, nodes)]``: consecutive output ranges whose node closures
    hold at most ``max_live`` values (one output may exceed it alone).  With
    ``align`` > 1 every range but the last ends on a multiple of ``align``
    outputs where that leaves it non-empty (the outputs past that multiple
    start the next range), so ranges of B columns meet on cache-line
    boundaries."""
    nodes = plan.nodes
    outs = plan.outputs
    chunks = []
    first = 0
    while first < len(outs):
        cur, cost, f = set(), 0, first
        while f < len(outs):
            new = _closure(nodes, outs[f][0], set()) - cur
            add = sum(nodes[n]["dim"] for n in new)
            if cur and cost + add > max_live:
                break
            cur |= new
            cost += add
            f += 1
        cut = f - f % align
        if f < len(outs) and first < cut < f:
            f = cut
            cur = set()
            for g in range(first, f):
                cur |= _closure(nodes, outs[g][0], set())
        chunks.append((first, f, cur))
        first = f
    return chunks


def _emit_tile_store(w, F, pitch, dtype, vector=True):
    """Write the staged [rows, F] tile (type OUT) to B[s0*F : (s0+rows)*F] (contiguous)."""
    vec = 4 if dtype == "f32" else 2
    vtype = "float4" if dtype == "f32" else "double2"
    w(f"    const long total = (long)rows * {F};")
    w(f"    OUT* __restrict__ dst = B + s0 * {F}L;")
    if pitch == F and not vector:
        # one element per lane and instruction: each store covers 64 consecutive values
        w("    #pragma unroll 8")
        w("    for (long i = lane; i < total; i += 64) dst[i] = st[i];")
    elif pitch == F:
        # flat copy; dst is 16-byte aligned when s0*F*sizeof(REAL) is (F*64*elem % 16 == 0)
        w(f"    if ((((unsigned long)dst) & 15) == 0) {{")
        w(f"      const long nv = total / {vec};")
        w(f"      const {vtype}* __restrict__ srcv = (const {vtype}*)st;")
        w(f"      {vtype}* __restrict__ dstv = ({vtype}*)dst;")
        w("      #pragma unroll 8")
        w("      for (long i = lane; i < nv; i += 64) dstv[i] = srcv[i];")
        w(f"      for (long i = nv * {vec} + lane; i < total; i += 64) dst[i] = st[i];")
        w("    } else {")
        w("      #pragma unroll 8")
        w("      for (long i = lane; i < total; i += 64) dst[i] = st[i];")
        w("    }")
    else:
        w("    #pragma unroll 8")
        w(f"    for (long i = lane; i < total; i += 64) {{ const long r = i / {F}; dst[i] = st[r * {pitch} + (i - r * {F})]; }}")


# LDS of a compute unit: a tile that fits a quarter of it lets four one-wave
# workgroups (one per SIMD) run on each CU
CU_LDS_BYTES = 160 * 1024


def tile_rows(F, out_dtype, rows=None):
    """Samples per workgroup: 64, or fewer when that lets one more tile fit per CU."""
    if rows is not None:
        return int(rows)
    elem = 8 if out_dtype == "f64" else 4
    pitch = F if F % 2 else F + 1
    fit64 = CU_LDS_BYTES // (64 * pitch * elem)
    for r in range(63, 55, -1):
        if CU_LDS_BYTES // (r * pitch * elem) > fit64 and CU_LDS_BYTES // (r * pitch * elem) <= 4:
            return r
    return 64


def _emit_node_code(w, nodes, n, emitted, dtype, src, lit=None):
    """Emit node ``n`` (and its dependencies) as straight-line register code.

    ``src(c)`` is the expression of density column ``c`` of the sample and
    ``lit(value)`` that of a coefficient (default: an instruction literal).
    """
    if lit is None:
        lit = lambda value: _lit(value, dtype)  # noqa: E731
    if n in emitted:
        return
    nd = nodes[n]
    for d in nd["deps"]:
        _emit_node_code(w, nodes, d, emitted, dtype, src, lit)
    emitted.add(n)
    fma = "fma" if dtype == "f64" else "fmaf"
    if nd["kind"] == "leaf":
        for c in range(nd["dim"]):
            w(f"      const REAL v{n}_{c} = {src(nd['a_offset'] + c)};")
        return
    per = [[] for _ in range(nd["dim"])]
    if nd["kind"] == "sym":
        srcn = nd["deps"][0]
        for oc, value, factors in nd["terms"]:
            per[oc].append((value, tuple(f"v{srcn}_{q}" for q in factors)))
    else:
        da, db = nd["deps"]
        for oc, value, (i, j) in nd["terms"]:
            per[oc].append((value, (f"v{da}_{i}", f"v{db}_{j}")))
    for c, terms in enumerate(per):
        if not terms:
            w(f"      const REAL v{n}_{c} = (REAL)0;")
            continue
        groups = {}
        for value, fac in terms:
            groups.setdefault(fac[0], []).append((value, fac[1:]))
        # sum_head head * (sum c * tail), as up to CHAINS independent fma chains
        # added at the end (instruction-level parallelism for one wave per SIMD)
        chains = [None] * min(CHAINS, len(groups))
        for g, (head, rest) in enumerate(groups.items()):
            inner = None
            for value, tail in rest:
                prod = " * ".join(tail) if tail else "(REAL)1"
                inner = (f"{lit(value)} * {prod}" if inner is None
                         else f"{fma}({lit(value)}, {prod}, {inner})")
            k = g % len(chains)
            chains[k] = f"{head} * ({inner})" if chains[k] is None else f"{fma}({head}, {inner}, {chains[k]})"
        while len(chains) > 1:
            chains = [f"({chains[i]} + {chains[i + 1]})" if i + 1 < len(chains) else chains[i]
                      for i in range(0, len(chains), 2)]
        w(f"      const REAL v{n}_{c} = {chains[0]};")


def _emit_one_chain(w, nodes, n, emitted, dtype, leaf, indent="    "):
    """Emit node ``n`` (and its dependencies) as straight-line register code,
    one fma chain per component: terms grouped by their first factor,
    ``sum_a x_a * (sum c * rest)``.  ``leaf(c)`` is the expression of density
    column ``c``.  The generated parts and their fused readout share it, so a
    feature has the same bits in both."""
    if n in emitted:
        return
    nd = nodes[n]
    for d in nd["deps"]:
        _emit_one_chain(w, nodes, d, emitted, dtype, leaf, indent)
    emitted.add(n)
    fma = "fma" if dtype == "f64" else "fmaf"
    if nd["kind"] == "leaf":
        for c in range(nd["dim"]):
            w(f"{indent}const REAL v{n}_{c} = {leaf(nd['a_offset'] + c)};")
        return
    per = [[] for _ in range(nd["dim"])]
    if nd["kind"] == "sym":
        src = nd["deps"][0]
        for oc, value, factors in nd["terms"]:
            per[oc].append((value, tuple(f"v{src}_{q}" for q in factors)))
    else:
        da, db = nd["deps"]
        for oc, value, (i, j) in nd["terms"]:
            per[oc].append((value, (f"v{da}_{i}", f"v{db}_{j}")))
    for c, terms in enumerate(per):
        if not terms:
            w(f"{indent}const REAL v{n}_{c} = (REAL)0;")
            continue
        groups = {}
        for value, fac in terms:
            groups.setdefault(fac[0], []).append((value, fac[1:]))
        parts = []
        for head, rest in groups.items():
            inner = None
            for value, tail in rest:
                prod = " * ".join(tail) if tail else "(REAL)1"
                inner = (f"{_lit(value, dtype)} * {prod}" if inner is None
                         else f"{fma}({_lit(value, dtype)}, {prod}, {inner})")
            parts.append((head, inner))
        expr = None
        for head, inner in parts:
            expr = f"{head} * ({inner})" if expr is None else f"{fma}({head}, {inner}, {expr})"
        w(f"{indent}const REAL v{n}_{c} = {expr};")


def _split_outputs(plan, parts):
    """Contiguous output ranges of about equal arithmetic (terms of the nodes
    each range computes, shared nodes counted in every range that needs them)."""
    nodes = plan.nodes

    def cost(nset):
        return sum(len(nodes[n].get("terms", ())) + nodes[n]["dim"] for n in nset)

    total = cost(set().union(*(_closure(nodes, r, set()) for r, _ in plan.outputs)))
    bounds, cur, first = [], set(), 0
    for f, (root, _c) in enumerate(plan.outputs):
        cur |= _closure(nodes, root, set())
        if len(bounds) < parts - 1 and cost(cur) >= total / parts and f + 1 < len(plan.outputs):
            bounds.append((first, f + 1))
            cur, first = set(), f + 1
    bounds.append((first, len(plan.outputs)))
    return bounds


def generate_persistent(plan, dtype="f32", out_dtype=None, kernel_name="ye3t_product_generated", waves=1,
                        store_policy=0, in_dtype=None):
    """Persistent variant of the single-chunk kernel: a workgroup loops over
    64-sample tiles ``blockIdx.x, blockIdx.x + gridDim.x, ...``.

    The next tile's density rows are requested before the current tile is
    computed, and a tile is stored by a fixed, fully unrolled sequence of
    16-byte buffer stores whose out-of-range lanes the hardware drops (the
    last tile is partial).  With that fixed count the
    compiler's wait for the next rows (issued before the stores) does not wait
    for the stores to drain, so the stores of tile i overlap the arithmetic of
    tile i + 1.  Requires an odd feature count (the tile is staged with row
    pitch F) and a 16-byte aligned ``B`` (the host uses the generic kernel
    otherwise).

    ``waves`` > 1: a workgroup of ``64 * waves`` threads shares the tile; wave
    w computes the w-th of ``waves`` contiguous output ranges of about equal
    arithmetic (fewer live values per wave), and all threads store the tile.

    ``store_policy``: cache-policy bits of the B stores (gfx950 buffer-store
    ``aux``: 1 = sc0, 2 = nt, 16 = sc1).

    ``in_dtype`` (default ``dtype``): type of the density rows; "f32" with an
    "f64" plan converts each value to fp64 as it is loaded.
    """
    out_dtype = out_dtype or dtype
    in_dtype = _check_in_dtype(dtype, in_dtype)
    if dtype == "f32" and out_dtype != "f32":
        raise ValueError("an f32 plan writes f32 features")
    real = "double" if dtype == "f64" else "float"
    outt = "double" if out_dtype == "f64" else "float"
    vec = 4 if out_dtype == "f32" else 2
    F, Wd = plan.feature_count, plan.a_width
    if F % 2 == 0:
        raise ValueError("the persistent kernel stages rows with pitch F, which must be odd")
    pitch = F
    nodes = plan.nodes
    out = []
    w = out.append
    w("// generated by ye3t_amd.ace.codegen (persistent) -- do not edit (compiled with hipRTC)")
    w(f"#define REAL {real}")
    w(f"#define OUT {outt}")
    w(f"#define AIN {_ctype(in_dtype)}")
    w("typedef unsigned v4u __attribute__((ext_vector_type(4)));")
    w("typedef unsigned v2u __attribute__((ext_vector_type(2)));")
    threads = 64 * waves
    w(f"extern \"C\" __global__ __launch_bounds__({threads}) void {kernel_name}(")
    w("    const AIN* __restrict__ A, long samples, OUT* __restrict__ B) {")
    w(f"  __shared__ __attribute__((aligned(16))) OUT st[64 * {pitch}];")
    w("  const int lane = threadIdx.x & 63;")
    w("  const int wv = threadIdx.x >> 6;")
    w("  const long tiles = (samples + 63) / 64;")
    w("  long tile = blockIdx.x;")
    w("  if (tile >= tiles) return;")
    w("  long srow = tile * 64 + lane;")
    w("  srow = srow < samples ? srow : samples - 1;")
    for c in range(Wd):
        w(f"  REAL a{c} = (REAL)A[srow * {Wd}L + {c}];")
    w("  for (;;) {")
    w("    const long next = tile + gridDim.x;")
    w("    long nrow = next * 64 + lane;")
    w("    nrow = nrow < samples ? nrow : samples - 1;")
    for c in range(Wd):
        w(f"    const AIN n{c} = A[nrow * {Wd}L + {c}];")
    for g, (f0, f1) in enumerate(_split_outputs(plan, waves)):
        w(f"    if (wv == {g}) {{" if waves > 1 else "    {")
        emitted = set()
        for f in range(f0, f1):
            root, comp = plan.outputs[f]
            _emit_node_code(w, nodes, root, emitted, dtype, lambda c: f"a{c}")
            w(f"      st[lane * {pitch} + {f}] = (OUT)v{root}_{comp};")
        w("    }")
    w("    __syncthreads();")
    # fixed unrolled store of the [rows, F] tile (a contiguous block of B)
    # through a buffer resource sized to the tile: every lane stores on every
    # instruction (no branches, so the store count is known to the compiler)
    # and the hardware drops the stores of lanes past the tile's data
    total_full = 64 * F
    nv_full = total_full // vec
    iters = -(-nv_full // threads)
    esize = 8 if out_dtype == "f64" else 4
    w("    const long s0 = tile * 64;")
    w("    const long rem = samples - s0;")
    w("    const int rows = rem < 64 ? (int)rem : 64;")
    w(f"    const int total = rows * {F};")
    w(f"    const int nv = total / {vec};")
    w(f"    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)(B + s0 * {F}L), (short)0, "
      f"total * {esize}, 0x00020000);")
    w("    const v4u* __restrict__ srcv = (const v4u*)st;")
    for k in range(iters):
        w(f"    {{ const int j = threadIdx.x + {threads * k}; "
          f"__builtin_amdgcn_raw_buffer_store_b128(srcv[j < nv ? j : 0], rb, j < nv ? j * 16 : 0x7ffffff0, 0, "
          f"{int(store_policy)}); }}")
    if out_dtype == "f64":
        w(f"    {{ const int j = nv * {vec} + (int)threadIdx.x; __builtin_amdgcn_raw_buffer_store_b64("
          f"__builtin_bit_cast(v2u, st[j < total ? j : 0]), rb, j < total ? j * {esize} : 0x7ffffff0, 0, "
          f"{int(store_policy)}); }}")
    else:
        w(f"    {{ const int j = nv * {vec} + (int)threadIdx.x; __builtin_amdgcn_raw_buffer_store_b32("
          f"__builtin_bit_cast(unsigned, st[j < total ? j : 0]), rb, j < total ? j * {esize} : 0x7ffffff0, 0, "
          f"{int(store_policy)}); }}")
    w("    __syncthreads();")
    w("    if (next >= tiles) break;")
    w("    tile = next;")
    for c in range(Wd):
        w(f"    a{c} = (REAL)n{c};")
    w("  }")
    w("}")
    source = "\n".join(out) + "\n"
    meta = {"kernel": kernel_name, "chunks": 1, "rows": 64, "persistent": True, "threads": threads,
            "feature_count": F,
            "a_width": Wd, "dtype": dtype, "out_dtype": out_dtype, "in_dtype": in_dtype,
            "hash": hashlib.sha256(source.encode()).hexdigest()[:16]}
    return source, meta


def generate_readout(plan, dtype="f32", out_dtype=None, kernel_name="ye3t_product_readout", waves=2,
                     in_dtype=None):
    """Fused linear readout ``out[s] = bias + sum_f W[f] B[s, f]`` without
    materialising B: the persistent tile loop of :func:`generate_persistent`
    (64 samples per tile, next tile's rows prefetched, ``waves`` waves sharing a
    tile over contiguous output ranges), where each wave folds its outputs into
    one fp-``dtype`` sum per sample as they are computed, in output order.  The
    wave sums and the bias are added in a fixed order (deterministic); one
    value per sample is stored.

    Kernel signature: ``(const AIN* A, long samples, OUT* out, const REAL* W, REAL bias)``
    (``AIN`` = ``in_dtype``, default ``dtype``).
    Counterpart of the reference's fused ``factorized_angular_linear``
    (``execution_plan_cuda.cu:8957``; readout semantics ``execution_plan.py:13832-13850``).
    """
    out_dtype = out_dtype or dtype
    in_dtype = _check_in_dtype(dtype, in_dtype)
    if dtype == "f32" and out_dtype != "f32":
        raise ValueError("an f32 plan writes f32 values")
    real = "double" if dtype == "f64" else "float"
    outt = "double" if out_dtype == "f64" else "float"
    fma = "fma" if dtype == "f64" else "fmaf"
    Wd = plan.a_width
    nodes = plan.nodes
    out = []
    w = out.append
    w("// generated by ye3t_amd.ace.codegen (fused linear readout) -- do not edit (compiled with hipRTC)")
    w(f"#define REAL {real}")
    w(f"#define OUT {outt}")
    w(f"#define AIN {_ctype(in_dtype)}")
    threads = 64 * waves
    w(f"extern \"C\" __global__ __launch_bounds__({threads}) void {kernel_name}(")
    w("    const AIN* __restrict__ A, long samples, OUT* __restrict__ out, const REAL* __restrict__ W, REAL bias) {")
    w(f"  __shared__ REAL part[{waves}][64];")
    w("  const int lane = threadIdx.x & 63;")
    w("  const int wv = threadIdx.x >> 6;")
    w("  const long tiles = (samples + 63) / 64;")
    w("  long tile = blockIdx.x;")
    w("  if (tile >= tiles) return;")
    w("  long srow = tile * 64 + lane;")
    w("  srow = srow < samples ? srow : samples - 1;")
    for c in range(Wd):
        w(f"  REAL a{c} = (REAL)A[srow * {Wd}L + {c}];")
    w("  for (;;) {")
    w("    const long next = tile + gridDim.x;")
    w("    long nrow = next * 64 + lane;")
    w("    nrow = nrow < samples ? nrow : samples - 1;")
    for c in range(Wd):
        w(f"    const AIN n{c} = A[nrow * {Wd}L + {c}];")
    for g, (f0, f1) in enumerate(_split_outputs(plan, waves)):
        w(f"    if (wv == {g}) {{" if waves > 1 else "    {")
        w("      REAL acc = (REAL)0;")
        emitted = set()
        for f in range(f0, f1):
            root, comp = plan.outputs[f]
            _emit_node_code(w, nodes, root, emitted, dtype, lambda c: f"a{c}")
            w(f"      acc = {fma}(W[{f}], v{root}_{comp}, acc);")
        w(f"      part[{g}][lane] = acc;")
        w("    }")
    w("    __syncthreads();")
    w("    if (wv == 0) {")
    w("      REAL r = bias;")
    for g in range(waves):
        w(f"      r += part[{g}][lane];")
    w("      const long s = tile * 64 + lane;")
    w("      if (s < samples) out[s] = (OUT)r;")
    w("    }")
    w("    __syncthreads();")
    w("    if (next >= tiles) break;")
    w("    tile = next;")
    for c in range(Wd):
        w(f"    a{c} = (REAL)n{c};")
    w("  }")
    w("}")
    src = "\n".join(out) + "\n"
    meta = {"kernel": kernel_name, "threads": threads, "feature_count": plan.feature_count, "a_width": Wd,
            "dtype": dtype, "out_dtype": out_dtype, "in_dtype": in_dtype,
            "hash": hashlib.sha256(src.encode()).hexdigest()[:16]}
    return src, meta


def generate_adjoint(plan, dtype="f64", grad_dtype=None, kernel_name="ye3t_product_adjoint", waves=2,
                     in_dtype=None):
    """Reverse mode of the product: ``gA[s] = J(A[s])^T gB[s]`` (counterpart of
    the reference's ``factorized_angular_adjoint``, ``execution_plan_cuda.cu:6361``;
    CPU core ``ye3t_runtime_core.h:1431-1456``).

    Persistent over 64-sample tiles.  The tile's output gradients (``gB``, of
    ``grad_dtype``, default ``dtype``; 16-byte aligned) are loaded into LDS with
    contiguous 16-byte loads, all issued before the first LDS write.
    The adjoint is linear in gB, so wave w handles the w-th of ``waves`` output
    ranges: it recomputes the forward values its range depends on, then sweeps
    the nodes in reverse creation order (dependencies are created first)
    accumulating node adjoints with the product rule, and leaves its partial
    density gradient in LDS.  The partials are added in wave order (fixed) and
    the ``[rows, a_width]`` block of gA is stored with contiguous stores.

    Kernel signature: ``(const AIN* A, const GT* gB, long samples, AIN* gA)``:
    the density and its gradient have the type ``in_dtype`` (default ``dtype``);
    the arithmetic is ``dtype``.
    """
    grad_dtype = grad_dtype or dtype
    in_dtype = _check_in_dtype(dtype, in_dtype)
    if dtype == "f32" and grad_dtype != "f32":
        raise ValueError("an f32 plan takes f32 gradients")
    real = "double" if dtype == "f64" else "float"
    gt = "double" if grad_dtype == "f64" else "float"
    fma = "fma" if dtype == "f64" else "fmaf"
    F, Wd = plan.feature_count, plan.a_width
    pitch = F if F % 2 else F + 1
    nodes = plan.nodes
    out = []
    w = out.append
    w("// generated by ye3t_amd.ace.codegen (product adjoint) -- do not edit (compiled with hipRTC)")
    w(f"#define REAL {real}")
    w(f"#define GT {gt}")
    w(f"#define AIN {_ctype(in_dtype)}")
    threads = 64 * waves
    w(f"extern \"C\" __global__ __launch_bounds__({threads}) void {kernel_name}(")
    w("    const AIN* __restrict__ A, const GT* __restrict__ gB, long samples, AIN* __restrict__ gA) {")
    w(f"  __shared__ __attribute__((aligned(16))) GT gt[64 * {pitch}];")
    w(f"  __shared__ REAL gp[{waves}][{Wd}][64];")
    w("  const int lane = threadIdx.x & 63;")
    w("  const int wv = threadIdx.x >> 6;")
    w("  const long tiles = (samples + 63) / 64;")
    w("  for (long tile = blockIdx.x; tile < tiles; tile += gridDim.x) {")
    w("    const long s0 = tile * 64;")
    w("    const int rows = samples - s0 < 64 ? (int)(samples - s0) : 64;")
    if pitch == F:
        # the LDS tile is the contiguous [rows, F] block of gB: every 16-byte
        # load of the block is issued before the first LDS write (one memory
        # latency per tile), then a scalar tail for a partial tile
        ve = 16 // (8 if grad_dtype == "f64" else 4)
        vt = "double" if grad_dtype == "f64" else "float"
        iters = -(-(64 * F // ve) // threads)
        w(f"    typedef {vt} gv __attribute__((ext_vector_type({ve})));")
        w(f"    const int nv = rows * {F} / {ve};")
        w(f"    const gv* __restrict__ src = (const gv*)(gB + s0 * {F}L);")
        for k in range(iters):
            w(f"    const int j{k} = threadIdx.x + {threads * k};")
            w(f"    const gv t{k} = src[j{k} < nv ? j{k} : 0];")
        for k in range(iters):
            w(f"    if (j{k} < nv) ((gv*)gt)[j{k}] = t{k};")
        w(f"    for (int i = nv * {ve} + (int)threadIdx.x; i < rows * {F}; i += {threads}) gt[i] = gB[s0 * {F}L + i];")
    else:
        w(f"    for (int i = threadIdx.x; i < rows * {F}; i += {threads}) {{")
        w(f"      const int r = i / {F};")
        w(f"      gt[r * {pitch} + (i - r * {F})] = gB[s0 * {F}L + i];")
        w("    }")
    w("    const long srow = s0 + (lane < rows ? lane : rows - 1);")
    for c in range(Wd):
        w(f"    const REAL a{c} = (REAL)A[srow * {Wd}L + {c}];")
    w("    __syncthreads();")
    for g, (f0, f1) in enumerate(_split_outputs(plan, waves)):
        w(f"    if (wv == {g}) {{" if waves > 1 else "    {")
        roots = sorted({plan.outputs[f][0] for f in range(f0, f1)})
        needed = set()
        for r in roots:
            _closure(nodes, r, needed)
        emitted = set()
        for r in roots:
            for d in nodes[r]["deps"]:
                _emit_node_code(w, nodes, d, emitted, dtype, lambda c: f"a{c}")
        # adjoint accumulators: output components start from the gradient tile
        init = {}
        for f in range(f0, f1):
            root, comp = plan.outputs[f]
            init[(root, comp)] = f"(REAL)gt[lane * {pitch} + {f}]"
        for n in sorted(needed):
            for c in range(nodes[n]["dim"]):
                w(f"      REAL g{n}_{c} = {init.get((n, c), '(REAL)0')};")
        for n in sorted(needed, reverse=True):
            nd = nodes[n]
            if nd["kind"] == "leaf":
                continue
            if nd["kind"] == "pair":
                da, db = nd["deps"]
                for oc, value, (i, j) in nd["terms"]:
                    cg = f"({_lit(value, dtype)} * g{n}_{oc})"
                    w(f"      g{da}_{i} = {fma}({cg}, v{db}_{j}, g{da}_{i});")
                    w(f"      g{db}_{j} = {fma}({cg}, v{da}_{i}, g{db}_{j});")
            else:
                srcn = nd["deps"][0]
                for oc, value, factors in nd["terms"]:
                    cg = f"({_lit(value, dtype)} * g{n}_{oc})"
                    for m, q in enumerate(factors):
                        rest = [f"v{srcn}_{x}" for k2, x in enumerate(factors) if k2 != m]
                        prod = " * ".join(rest) if rest else "(REAL)1"
                        w(f"      g{srcn}_{q} = {fma}({cg}, {prod}, g{srcn}_{q});")
        touched = {}
        for n in sorted(needed):
            nd = nodes[n]
            if nd["kind"] == "leaf":
                for c in range(nd["dim"]):
                    touched[nd["a_offset"] + c] = f"g{n}_{c}"
        for col in range(Wd):
            w(f"      gp[{g}][{col}][lane] = {touched.get(col, '(REAL)0')};")
        w("    }")
    w("    __syncthreads();")
    w(f"    for (int i = threadIdx.x; i < rows * {Wd}; i += {threads}) {{")
    w(f"      const int r = i / {Wd};")
    w(f"      const int col = i - r * {Wd};")
    w("      REAL v = gp[0][col][r];")
    for g in range(1, waves):
        w(f"      v += gp[{g}][col][r];")
    w(f"      gA[s0 * {Wd}L + i] = (AIN)v;")
    w("    }")
    w("    __syncthreads();")
    w("  }")
    w("}")
    src = "\n".join(out) + "\n"
    meta = {"kernel": kernel_name, "threads": threads, "feature_count": F, "a_width": Wd, "dtype": dtype,
            "grad_dtype": grad_dtype, "in_dtype": in_dtype, "hash": hashlib.sha256(src.encode()).hexdigest()[:16]}
    return src, meta


def generate(plan, dtype="f32", max_live=None, kernel_name="ye3t_product_generated", out_dtype=None, rows=None,
             in_dtype=None, chunks=None, strided=False, group=GROUP):
    """Return ``(source, meta)`` for a specialised product kernel.

    ``dtype`` is the type of ``A`` and of the arithmetic, ``out_dtype`` (default
    the same; "f32" with an "f64" plan) that of ``B``.  ``rows`` (<= 64,
    default :func:`tile_rows`) is the number of samples a 64-lane workgroup
    produces; lanes past it idle.  ``in_dtype`` (default ``dtype``) is the
    storage type of ``A`` ("f32" with an "f64" plan: converted as loaded).
    ``chunks`` (default: the plan's chunks at ``max_live``) restricts the
    kernel to those output chunks, one per grid row, with 64-sample tiles
    (see :func:`generate_parts`).  ``strided``: the kernel takes two more
    arguments ``(row_stride, col_stride)`` and reads density value ``(s, k)``
    at ``A[s * row_stride + k * col_stride]``, so one code object serves the
    row-major density and its column-major copy.
    """
    out_dtype = out_dtype or dtype
    in_dtype = _check_in_dtype(dtype, in_dtype)
    if dtype == "f32" and out_dtype != "f32":
        raise ValueError("an f32 plan writes f32 features")
    real = "double" if dtype == "f64" else "float"
    outt = "double" if out_dtype == "f64" else "float"
    fma = "fma" if dtype == "f64" else "fmaf"
    if max_live is None:
        max_live = 1 << 30  # one chunk unless asked otherwise
    nodes = plan.nodes
    # a kernel restricted to given chunks always uses 64-row tiles and writes its columns only
    single = chunks is None
    if chunks is None:
        chunks = _chunks(plan, max_live)
    F = plan.feature_count
    out = []
    w = out.append
    w("// generated by ye3t_amd.ace.codegen -- do not edit (compiled with hipRTC)")
    w(f"#define REAL {real}")
    w(f"#define OUT {outt}")
    w(f"#define AIN {_ctype(in_dtype)}")
    if strided:
        w("typedef unsigned v2u __attribute__((ext_vector_type(2)));")
    w(f"extern \"C\" __global__ __launch_bounds__(64) void {kernel_name}(")
    if strided:
        # density value (s, k) at A[s * row_stride + k * col_stride]: rows (a_width, 1) or columns (1, ld)
        w("    const AIN* __restrict__ A, long samples, OUT* __restrict__ B, long row_stride, long col_stride) {")
    else:
        w("    const AIN* __restrict__ A, long samples, OUT* __restrict__ B) {")
    single = single and len(chunks) == 1
    R = tile_rows(F, out_dtype, rows) if single else 64
    if not 1 <= R <= 64:
        raise ValueError("rows per tile must be in [1, 64]")
    pitch = F if F % 2 else F + 1  # odd row pitch of the staged tile
    if single:
        w(f"  __shared__ __attribute__((aligned(16))) OUT st[{R} * {pitch}];")
    else:
        w(f"  __shared__ OUT st[{group}][65];")
    w("  const int lane = threadIdx.x;")
    if strided:
        # XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by
        # linear id, so XCD x gets the tiles [x * per, (x + 1) * per) of every
        # chunk (gridDim.x = 8 * per, gridDim.y = the part's chunks); on an XCD
        # the chunks of one tile run back to back, so the tile's density rows
        # are read from HBM once per part and then from L2
        w("  const long wg = (long)blockIdx.y * gridDim.x + blockIdx.x;")
        w("  const long per = gridDim.x >> 3, k = wg >> 3;")
        w("  const long tile = (wg & 7) * per + k / gridDim.y;")
        w("  const int chunk = (int)(k % gridDim.y);")
        w(f"  const long s0 = tile * {R};")
        w("  if (s0 >= samples) return;")
    else:
        w(f"  const long s0 = (long)blockIdx.x * {R};")
    w("  const long s = s0 + lane;")
    w(f"  const bool valid = lane < {R} && s < samples;")
    if strided:
        # wave-uniform tile bases and 32-bit byte offsets of the lane (the host
        # keeps 63 * row_stride elements and a tile of B below 4 GiB): a density
        # load is one global_load from the column's address in SGPRs plus the
        # lane's offset, a store likewise, with no 64-bit address arithmetic
        w("  const char* __restrict__ at = (const char*)(A + s0 * row_stride);")
        w("  const long cs = col_stride * (long)sizeof(AIN);")
        w("  const unsigned alane = (unsigned)(valid ? lane : 0) * (unsigned)(row_stride * (long)sizeof(AIN));")
        w(f"  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)(B + s0 * {F}L), (short)0, "
          f"{64 * F * (8 if out_dtype == 'f64' else 4)}, 0x00020000);")
    else:
        w(f"  const AIN* __restrict__ a = A + (valid ? s : 0) * {plan.a_width}L;")
    w("  const long rem = samples - s0;")
    w(f"  const int rows = rem < {R} ? (int)rem : {R};")
    w("  switch (chunk) {" if strided else "  switch (blockIdx.y) {")
    for ci, (first, last, members) in enumerate(chunks):
        w(f"  case {ci}: {{")
        emitted = set()

        # unconditional loads: lanes past the last sample read sample 0 (a valid
        # address) and their outputs are never stored; a select per load would
        # turn each into a branch that waits for its own data
        leaf = ((lambda c: f"(REAL)*(const AIN*)(at + {c}L * cs + alane)") if strided
                else (lambda c: f"(REAL)a[{c}]"))

        def emit(n):
            _emit_one_chain(w, nodes, n, emitted, dtype, leaf)

        if strided:
            # every density value of the chunk requested up front (independent loads in flight together)
            for n in sorted((m for m in members if nodes[m]["kind"] == "leaf"), key=lambda m: nodes[m]["a_offset"]):
                emit(n)
        if single:
            for f in range(first, last):
                root, comp = plan.outputs[f]
                emit(root)
                stmt = f"st[lane * {pitch} + {f}] = (OUT)v{root}_{comp};"
                w(f"    {stmt}" if R == 64 else f"    if (lane < {R}) {stmt}")
            w("    __syncthreads();")
            # 16-byte stores need every tile's block of B 16-byte aligned
            out_elem = 8 if out_dtype == "f64" else 4
            _emit_tile_store(w, F, pitch, out_dtype, vector=(R * F * out_elem) % 16 == 0)
            w("    break;")
            w("  }")
            continue
        for g0 in range(first, last, group):
            g1 = min(g0 + group, last)
            for f in range(g0, g1):
                root, comp = plan.outputs[f]
                emit(root)
                w(f"    st[{f - g0}][lane] = (OUT)v{root}_{comp};")
            width = g1 - g0
            w("    __syncthreads();")
            if strided:
                # a full tile: the [64, width] block as `width` stores of 64
                # consecutive row-major elements, LDS reads issued in batches
                # ahead of their stores (no loop, no wait per element)
                out_elem = 8 if out_dtype == "f64" else 4
                if out_elem == 8:
                    store = "__builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, {v}), rb, {vo}, {so}, 0);"
                else:
                    store = "__builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, {v}), rb, {vo}, {so}, 0);"
                w("    if (rows == 64) {")
                if 64 % width == 0:
                    # store k covers rows r0 + k * 64 / width: constant LDS
                    # offsets and a constant scalar offset into B's tile
                    step = 64 // width
                    w(f"      const int r0 = lane / {width}, c0 = lane - r0 * {width};")
                    w("      const OUT* sp = &st[c0][r0];")
                    w(f"      const unsigned u0 = (unsigned)(r0 * {F} + {g0} + c0) * {out_elem}u;")
                for b0 in range(0, width, STORE_BATCH):
                    b1 = min(b0 + STORE_BATCH, width)
                    w("    {")
                    for k in range(b0, b1):
                        if 64 % width == 0:
                            w(f"      const OUT o{k} = sp[{k * step}];")
                        else:
                            w(f"      const int i{k} = lane + {64 * k}, r{k} = i{k} / {width}, "
                              f"c{k} = i{k} - r{k} * {width};")
                            w(f"      const OUT o{k} = st[c{k}][r{k}];")
                    for k in range(b0, b1):
                        if 64 % width == 0:
                            w("      " + store.format(v=f"o{k}", vo="u0", so=f"{k * step * F * out_elem}"))
                        else:
                            w("      " + store.format(v=f"o{k}", vo=f"(unsigned)(r{k} * {F} + {g0} + c{k}) * {out_elem}u",
                                                      so="0"))
                    w("    }")
                w("    } else {")
            w(f"    for (int i = lane; i < rows * {width}; i += 64) {{")
            w(f"      const int r = i / {width}, c = i - r * {width};")
            w(f"      B[(s0 + r) * {F}L + {g0} + c] = st[c][r];")
            w("    }")
            if strided:
                w("    }")
            w("    __syncthreads();")
        w("    break;")
        w("  }")
    w("  default: break;")
    w("  }")
    w("}")
    source = "\n".join(out) + "\n"
    meta = {"kernel": kernel_name, "chunks": len(chunks), "rows": R, "feature_count": F, "a_width": plan.a_width,
            "dtype": dtype, "out_dtype": out_dtype, "in_dtype": in_dtype, "first_output": chunks[0][0],
            "last_output": chunks[-1][1], "strided": bool(strided),
            "hash": hashlib.sha256(source.encode()).hexdigest()[:16]}
    return source, meta


# node values per chunk of a generated part and chunks per part: config 2 (fp64)
# measured 127 us at (400, 9), 135 us at (400, 6), 140 us at (300, 6), 162 us at
# (500, 4) and 216 us at (800, 2); larger chunks re-read fewer density columns and
# recompute fewer shared nodes until they spill
PART_MAX_LIVE = 400
PART_CHUNKS = 9
# plans above PART_LARGE_TERMS terms in fp64 arithmetic take 300-value chunks:
# config 3 (fp64) 3.67 ms at (300, 9) against 4.06 ms at (400, 9), 3.95 at
# (400, 16), 4.23 at (400, 5) and 4.69 at (500, 9); config 5 (fp64 arithmetic)
# 158 ms against 174 ms.  In fp32 arithmetic (half the registers per value)
# config 3 took 1.85 ms at 300 against 1.72 ms at 400.
PART_MAX_LIVE_LARGE = 300
PART_LARGE_TERMS = 100_000


# plans above PART_LARGE_TERMS terms take 64 chunks per part: each part reads a
# tile's density rows from HBM once, so fewer parts re-read less (config 3 fp64
# 3.49 / 3.27 / 3.00 / 2.86 ms at 9 / 16 / 32 / 64 chunks per part, config 5
# 129 / 126 / 118 / 113 ms; a 64-chunk part compiles in about a minute)
PART_CHUNKS_LARGE = 64


def _plan_terms(plan):
    return sum(len(nd.get("terms", ())) for nd in plan.nodes)


def part_chunks(plan):
    """Chunks per generated part of ``plan``."""
    return PART_CHUNKS_LARGE if _plan_terms(plan) > PART_LARGE_TERMS else PART_CHUNKS


def part_max_live(plan, dtype="f64"):
    """Node values per chunk of the generated parts of ``plan`` in ``dtype`` arithmetic."""
    return PART_MAX_LIVE_LARGE if dtype == "f64" and _plan_terms(plan) > PART_LARGE_TERMS else PART_MAX_LIVE


def generate_parts(plan, dtype="f64", max_live=None, chunks_per_part=None, out_dtype=None,
                   in_dtype=None, group=GROUP):
    """``[(source, meta), ...]``: the plan's generated product kernel cut into
    parts of ``chunks_per_part`` consecutive output chunks (each chunk holds
    at most ``max_live`` node values), for plans whose code is too large for
    one hipRTC module (compile time grows faster than the code: 221 s for
    config 2's 16 810 terms as one kernel at 126 chunks, ~5 s per 9-chunk
    part of 400-value chunks).  Part i
    writes columns ``[meta["first_output"], meta["last_output"])`` of B; the
    parts run in order (``ye3t_hip_product_plan_attach_generated_parts``) and
    read the density through row and column strides (``strided``), so the
    column-major copy the interpreter reads serves them too: a leaf of 64
    samples is then one contiguous 512-byte load instead of 64 cache lines."""
    chunks_per_part = chunks_per_part or part_chunks(plan)
    if chunks_per_part < 1:
        raise ValueError("chunks_per_part must be positive")
    if 64 * plan.feature_count * (8 if (out_dtype or dtype) == "f64" else 4) >= 1 << 32:
        raise ValueError("a 64-sample tile of B must stay below 4 GiB for the generated parts")
    max_live = max_live or part_max_live(plan, dtype)
    # where every row of B starts on a 128-byte line, chunks end on line
    # boundaries: no line of B is then written in part by two workgroups
    # (config 3 fp64 stage 2 2.49 -> 1.87 ms, fp32 1.31 -> 0.99 ms, with 18 %
    # more chunks)
    out_elem = 8 if (out_dtype or dtype) == "f64" else 4
    align = 128 // out_elem if (plan.feature_count * out_elem) % 128 == 0 else 1
    chunks = _chunks(plan, max_live, align)
    parts = []
    for i in range(0, len(chunks), chunks_per_part):
        parts.append(generate(plan, dtype, max_live, kernel_name="ye3t_product_part", out_dtype=out_dtype,
                              in_dtype=in_dtype, chunks=chunks[i:i + chunks_per_part], strided=True,
                              group=group))
    return parts


def generate_adjoint_parts(plan, dtype="f64", max_live=PART_MAX_LIVE, chunks_per_part=PART_CHUNKS, grad_dtype=None,
                           in_dtype=None, group=GROUP):
    """Reverse mode of a plan too large for one module, in parts:
    ``gA[s] = J(A[s])^T gB[s]`` (counterpart of the reference's
    ``factorized_angular_adjoint``, ``execution_plan_cuda.cu:6361``).

    Chunks and parts are formed as in :func:`generate_parts`, without its
    alignment of chunk ends to lines of B (nothing here writes B).  For each tile
    of 64 samples a chunk recomputes the forward values its outputs depend on
    (density read through row and column strides), loads its outputs'
    gradients from ``gB`` (row segments staged through LDS, ``group`` columns
    at a time), sweeps its nodes in reverse creation order and writes the
    gradients of the density columns it touches as rows of a partial buffer
    ``P`` (``P[row * ldp + s]``, one row per (chunk, touched column)).  A
    reduction then sums, for each density column, its partial rows in chunk
    order (fixed, so the result does not depend on scheduling).

    Returns ``(parts, reduction)``: ``parts`` is ``[(source, meta), ...]`` with
    kernel signature ``(const AIN* A, const GT* gB, long samples, REAL* P,
    long row_stride, long col_stride, long ldp)``; ``reduction`` holds
    ``partial_rows`` (rows of ``P``), ``col_off`` (``[a_width + 1]``) and
    ``rows``: column ``k``'s partial rows are ``rows[col_off[k]:col_off[k + 1]]``.
    """
    import numpy as np

    grad_dtype = grad_dtype or dtype
    in_dtype = _check_in_dtype(dtype, in_dtype)
    if dtype == "f32" and grad_dtype != "f32":
        raise ValueError("an f32 plan takes f32 gradients")
    if chunks_per_part < 1:
        raise ValueError("chunks_per_part must be positive")
    if 64 * plan.feature_count * (8 if grad_dtype == "f64" else 4) >= 1 << 32:
        raise ValueError("a 64-sample tile of gB must stay below 4 GiB for the adjoint parts")
    real = "double" if dtype == "f64" else "float"
    gt = "double" if grad_dtype == "f64" else "float"
    fma = "fma" if dtype == "f64" else "fmaf"
    nodes = plan.nodes
    F, Wd = plan.feature_count, plan.a_width
    chunks = _chunks(plan, max_live)
    touched = []
    for _first, _last, members in chunks:
        touched.append(sorted(nodes[n]["a_offset"] + c for n in members if nodes[n]["kind"] == "leaf"
                              for c in range(nodes[n]["dim"])))
    row_base = [0]
    for cols in touched:
        row_base.append(row_base[-1] + len(cols))
    col_rows = [[] for _ in range(Wd)]
    for ci, cols in enumerate(touched):
        for j, k in enumerate(cols):
            col_rows[k].append(row_base[ci] + j)
    col_off = np.zeros(Wd + 1, dtype=np.int64)
    col_off[1:] = np.cumsum([len(r) for r in col_rows])
    rows = np.array([r for rs in col_rows for r in rs], dtype=np.int64)

    parts = []
    for p0 in range(0, len(chunks), chunks_per_part):
        sub = list(range(p0, min(len(chunks), p0 + chunks_per_part)))
        out = []
        w = out.append
        w("// generated by ye3t_amd.ace.codegen (product adjoint part) -- do not edit (compiled with hipRTC)")
        w(f"#define REAL {real}")
        w(f"#define GT {gt}")
        w(f"#define AIN {_ctype(in_dtype)}")
        w("typedef unsigned v2u __attribute__((ext_vector_type(2)));")
        w("extern \"C\" __global__ __launch_bounds__(64) void ye3t_product_adjoint_part(")
        w("    const AIN* __restrict__ A, const GT* __restrict__ gB, long samples, REAL* __restrict__ P,")
        w("    long row_stride, long col_stride, long ldp) {")
        w(f"  __shared__ GT st[{group}][65];")
        w("  const int lane = threadIdx.x;")
        # the forward parts' XCD-aware (tile, chunk) order
        w("  const long wg = (long)blockIdx.y * gridDim.x + blockIdx.x;")
        w("  const long per = gridDim.x >> 3, k = wg >> 3;")
        w("  const long tile = (wg & 7) * per + k / gridDim.y;")
        w("  const int chunk = (int)(k % gridDim.y);")
        w("  const long s0 = tile * 64;")
        w("  if (s0 >= samples) return;")
        w("  const long s = s0 + lane;")
        # scalar bases and 32-bit lane offsets, as in the forward parts: the
        # density column's address, the tile's rows of gB (a buffer resource)
        # and the partial row's address sit in SGPRs (the host keeps the
        # offsets below 4 GiB)
        w("  const char* __restrict__ at = (const char*)(A + s0 * row_stride);")
        w("  const long cs = col_stride * (long)sizeof(AIN);")
        w("  const unsigned alane = (unsigned)(s < samples ? lane : 0) * (unsigned)(row_stride * (long)sizeof(AIN));")
        w(f"  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc((void*)(gB + s0 * {F}L), (short)0, "
          f"{64 * F * (8 if grad_dtype == 'f64' else 4)}, 0x00020000);")
        w("  char* __restrict__ pt = (char*)(P + s0);")
        w("  const long pb = ldp * (long)sizeof(REAL);")
        w("  const unsigned plane = (unsigned)lane * (unsigned)sizeof(REAL);")
        w("  const long rem = samples - s0;")
        w("  const int rows = rem < 64 ? (int)rem : 64;")
        w("  switch (chunk) {")
        for lc, ci in enumerate(sub):
            first, last, members = chunks[ci]
            w(f"  case {lc}: {{")
            emitted = set()
            aleaf = lambda c: f"(REAL)*(const AIN*)(at + {c}L * cs + alane)"  # noqa: E731
            # every density value of the chunk, unconditionally (lanes past the
            # last sample read sample 0 and write only partial rows never summed)
            for n in sorted((m for m in members if nodes[m]["kind"] == "leaf"), key=lambda m: nodes[m]["a_offset"]):
                _emit_node_code(w, nodes, n, emitted, dtype, aleaf)
            roots = sorted({plan.outputs[f][0] for f in range(first, last)})
            needed = set()
            for r in roots:
                _closure(nodes, r, needed)
            for r in roots:
                for d in nodes[r]["deps"]:
                    _emit_node_code(w, nodes, d, emitted, dtype, aleaf)
            for n in sorted(needed):
                for c in range(nodes[n]["dim"]):
                    w(f"      REAL g{n}_{c} = (REAL)0;")
            # the chunk's output gradients, `group` columns at a time: a fixed,
            # unrolled set of loads (rows past the tile re-read its last row),
            # all issued before the LDS writes
            for g0 in range(first, last, group):
                g1 = min(g0 + group, last)
                width = g1 - g0
                w("      __syncthreads();")
                w("      {")
                w(f"        GT t[{width}];")
                gsz = 8 if grad_dtype == "f64" else 4
                load = ("__builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rg, {vo}, {so}, 0))"
                        if gsz == 8 else
                        "__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, {vo}, {so}, 0))")
                if 64 % width == 0:
                    # load u covers rows r0 + u * 64 / width: a constant scalar
                    # offset on a full tile, the row clamped otherwise
                    step = 64 // width
                    w(f"        const int r0 = lane / {width}, c0 = lane - r0 * {width};")
                    w(f"        const unsigned u0 = (unsigned)(r0 * {F} + {g0} + c0) * {gsz}u;")
                    w("        if (rows == 64) {")
                    for u in range(width):
                        w("          t[" + str(u) + "] = " + load.format(vo="u0", so=f"{u * step * F * gsz}") + ";")
                    w("        } else {")
                    for u in range(width):
                        vo = f"(unsigned)(min(r0 + {u * step}, rows - 1) * {F} + {g0} + c0) * {gsz}u"
                        w("          t[" + str(u) + "] = " + load.format(vo=vo, so="0") + ";")
                    w("        }")
                else:
                    w("#pragma unroll")
                    w(f"        for (int u = 0; u < {width}; ++u) {{")
                    w(f"          const int i = lane + 64 * u, r = i / {width}, c = i - r * {width};")
                    vo = f"(unsigned)((r < rows ? r : rows - 1) * {F} + {g0} + c) * {gsz}u"
                    w("          t[u] = " + load.format(vo=vo, so="0") + ";")
                    w("        }")
                w("#pragma unroll")
                w(f"        for (int u = 0; u < {width}; ++u) {{")
                w(f"          const int i = lane + 64 * u, r = i / {width}, c = i - r * {width};")
                w("          st[c][r] = t[u];")
                w("        }")
                w("      }")
                w("      __syncthreads();")
                for f in range(g0, g1):
                    root, comp = plan.outputs[f]
                    w(f"      g{root}_{comp} += (REAL)st[{f - g0}][lane];")
            for n in sorted(needed, reverse=True):
                nd = nodes[n]
                if nd["kind"] == "leaf":
                    continue
                if nd["kind"] == "pair":
                    da, db = nd["deps"]
                    for oc, value, (i, j) in nd["terms"]:
                        cg = f"({_lit(value, dtype)} * g{n}_{oc})"
                        w(f"      g{da}_{i} = {fma}({cg}, v{db}_{j}, g{da}_{i});")
                        w(f"      g{db}_{j} = {fma}({cg}, v{da}_{i}, g{db}_{j});")
                else:
                    srcn = nd["deps"][0]
                    for oc, value, factors in nd["terms"]:
                        cg = f"({_lit(value, dtype)} * g{n}_{oc})"
                        for m, q in enumerate(factors):
                            rest = [f"v{srcn}_{x}" for k2, x in enumerate(factors) if k2 != m]
                            prod = " * ".join(rest) if rest else "(REAL)1"
                            w(f"      g{srcn}_{q} = {fma}({cg}, {prod}, g{srcn}_{q});")
            leaf_of = {}
            for n in needed:
                if nodes[n]["kind"] == "leaf":
                    for c in range(nodes[n]["dim"]):
                        leaf_of[nodes[n]["a_offset"] + c] = f"g{n}_{c}"
            for j, col in enumerate(touched[ci]):
                w(f"      *(REAL*)(pt + {row_base[ci] + j}L * pb + plane) = {leaf_of.get(col, '(REAL)0')};")
            w("      break;")
            w("  }")
        w("  default: break;")
        w("  }")
        w("}")
        source = "\n".join(out) + "\n"
        meta = {"kernel": "ye3t_product_adjoint_part", "chunks": len(sub), "feature_count": F, "a_width": Wd,
                "dtype": dtype, "grad_dtype": grad_dtype, "in_dtype": in_dtype,
                "first_row": row_base[sub[0]], "last_row": row_base[sub[-1] + 1],
                "hash": hashlib.sha256(source.encode()).hexdigest()[:16]}
        parts.append((source, meta))
    return parts, {"partial_rows": row_base[-1], "col_off": col_off, "rows": rows}


def generate_readout_parts(plan, dtype="f64", max_live=None, chunks_per_part=None, in_dtype=None):
    """Fused linear readout of a plan in parts: ``out[s] = bias + sum_k B[s, k]
    weight[k]`` without writing B (counterpart of the reference's
    ``factorized_angular_linear``, ``execution_plan.py:13793-13850``).

    Chunks and parts are formed as in :func:`generate_parts`, without its
    alignment of chunk ends to lines of B (nothing here writes B), and a
    feature's emitted code is the forward's, so its value has the same bits
    however the outputs are chunked.  For each tile
    of 64 samples a chunk computes its outputs in registers (density through
    row and column strides) and writes ``sum_{k in chunk} weight[k] B[s, k]``
    to row ``chunk`` of a partial buffer ``P[chunk * ldp + s]``; the weights
    are read through the scalar cache.  A reduction adds the bias and the
    chunks' rows in chunk order.  Kernel signature: ``(const AIN* A, long
    samples, REAL* P, const REAL* W, long row_stride, long col_stride, long
    ldp)``.  Returns ``(parts, chunk_count)``.
    """
    in_dtype = _check_in_dtype(dtype, in_dtype)
    chunks_per_part = chunks_per_part or part_chunks(plan)
    if chunks_per_part < 1:
        raise ValueError("chunks_per_part must be positive")
    real = "double" if dtype == "f64" else "float"
    fma = "fma" if dtype == "f64" else "fmaf"
    nodes = plan.nodes
    F, Wd = plan.feature_count, plan.a_width
    chunks = _chunks(plan, max_live or part_max_live(plan, dtype))
    parts = []
    for p0 in range(0, len(chunks), chunks_per_part):
        sub = list(range(p0, min(len(chunks), p0 + chunks_per_part)))
        out = []
        w = out.append
        w("// generated by ye3t_amd.ace.codegen (readout part) -- do not edit (compiled with hipRTC)")
        w(f"#define REAL {real}")
        w(f"#define AIN {_ctype(in_dtype)}")
        w("typedef const __attribute__((address_space(4))) REAL* wptr;")
        w("extern \"C\" __global__ __launch_bounds__(64) void ye3t_product_readout_part(")
        w("    const AIN* __restrict__ A, long samples, REAL* __restrict__ P, const REAL* __restrict__ Wt,")
        w("    long row_stride, long col_stride, long ldp) {")
        w("  const int lane = threadIdx.x;")
        w("  const wptr W = (wptr)Wt;")
        w("  const long wg = (long)blockIdx.y * gridDim.x + blockIdx.x;")
        w("  const long per = gridDim.x >> 3, k = wg >> 3;")
        w("  const long tile = (wg & 7) * per + k / gridDim.y;")
        w("  const int chunk = (int)(k % gridDim.y);")
        w("  const long s0 = tile * 64;")
        w("  if (s0 >= samples) return;")
        w("  const long s = s0 + lane;")
        # density loads as in the forward parts: the column's address in SGPRs
        # plus the lane's 32-bit byte offset (the host keeps it below 4 GiB)
        w("  const char* __restrict__ at = (const char*)(A + s0 * row_stride);")
        w("  const long cs = col_stride * (long)sizeof(AIN);")
        w("  const unsigned alane = (unsigned)(s < samples ? lane : 0) * (unsigned)(row_stride * (long)sizeof(AIN));")
        w("  switch (chunk) {")
        for lc, ci in enumerate(sub):
            first, last, members = chunks[ci]
            w(f"  case {lc}: {{")
            emitted = set()
            leaf = lambda c: f"(REAL)*(const AIN*)(at + {c}L * cs + alane)"  # noqa: E731
            for n in sorted((m for m in members if nodes[m]["kind"] == "leaf"), key=lambda m: nodes[m]["a_offset"]):
                _emit_one_chain(w, nodes, n, emitted, dtype, leaf, "      ")
            # the chunk's dot product as CHAINS independent partial sums, added in a fixed
            # order; the features are computed exactly as the forward parts compute them
            names = [None] * min(CHAINS, last - first)
            for f in range(first, last):
                root, comp = plan.outputs[f]
                _emit_one_chain(w, nodes, root, emitted, dtype, leaf, "      ")
                j = (f - first) % len(names)
                prev = names[j]
                expr = f"W[{f}] * v{root}_{comp}" if prev is None else f"{fma}(W[{f}], v{root}_{comp}, {prev})"
                w(f"      const REAL r{j}_{f} = {expr};")
                names[j] = f"r{j}_{f}"
            total = names[0]
            for x in names[1:]:
                total = f"({total} + {x})"
            w(f"      P[{ci}L * ldp + s] = {total};")
            w("      break;")
            w("  }")
        w("  default: break;")
        w("  }")
        w("}")
        source = "\n".join(out) + "\n"
        meta = {"kernel": "ye3t_product_readout_part", "chunks": len(sub), "feature_count": F, "a_width": Wd,
                "dtype": dtype, "in_dtype": in_dtype, "first_chunk": sub[0],
                "hash": hashlib.sha256(source.encode()).hexdigest()[:16]}
        parts.append((source, meta))
    return parts, len(chunks)
