"""The replay adjoint with the forward kernel's scheduling: tm_adjoint as a persistent, step-refilled loop over a tape
in HBM (reference tallymap/_reverse.py:324-444, 1079-1180 is the adjoint it computes; reverse.py holds the shared
analysis: the PRE / LOOP / POST split, carry activity and relevance, the step, POST and PRE VJP programs).

Every lane runs one item at a time through three phases, one loop step per kernel iteration, and takes the next
item from the wave's claimed chunk as soon as it is free (the forward template's refill):

  count    the forward loop from the item's initial carries; the state before step k goes to tape slot k (slots
           0 .. TAPE-1 of the lane's own tape region); K = the number of steps.
  reverse  after POST and POST's VJP (the truncation flag, the cotangent lambda of the final carries), the steps
           newest first: state k from the tape, the step's VJP with lambda -> lambda, and the cotangents of the loop
           constants accumulated per item.
  finish   PRE's VJP: the per-item operand cotangents (stored) and one exact emit per differentiated broadcast
           element (reference _reverse.py:1172-1177).

Counting and reversing lanes share one code path: the step and its VJP form one program (the body replayed, its
transposes after it) whose primal outputs a counting lane keeps and whose cotangent outputs a reversing lane keeps;
a wave whose live lanes all count runs the plain step instead.  An item with K > TAPE steps takes the two-level
checkpointed sweep inside its lane (checkpoints every ceil(K / H) steps in the tape's first half H, each segment's
states in the second half, re-run from the checkpoint in pieces when longer than it).  The tape is the lane's
region of one buffer of launched lanes x TAPE x Wp u32 words, lane-major (word w of slot k of lane l at
(l * TAPE + k) * Wp + w; Wp = the state's words padded to a multiple of 4): under step refill a wave's lanes are at
different steps, so each lane's state is kept contiguous and its consecutive steps in consecutive 16-byte units;
nothing in it outlives the launch.
"""
import numpy as np

from .. import _ad as AD
from .. import _core as C
from . import kernel as K
from .codegen import Emitter, Val, VTally, assign_carries, ctype
from .reverse import ReverseError, plan

TAPE = 512                  # tape slots per lane: items with at most this many steps never recompute
REFILL = 32                 # free lanes a wave gathers before it takes items (measured: configs 3 and 5 on MI355X)

_W64 = {"i64", "u64", "double"}


def _nwords(dt):
    return 2 if ctype(dt) in _W64 else 1


def build(adj, block=K.BLOCK, tape=TAPE, chunk=K.CHUNK, refill=REFILL):
    """-> (HIP source, Layout) of the step-scheduled adjoint module (entry tm_adjoint).  refill: free lanes a wave
    waits for before it hands out items (64: the whole wave takes its next items together, which keeps its lanes in
    the same phase when items have similar lengths)."""
    prog = adj.prog
    nT, nP, nB = prog.nT, prog.nP, prog.nB
    pav, bav, yav = prog.p_avals(), prog.b_avals(), prog.y_avals()
    pl = plan(adj)
    sp, ft, fy = pl.sp, pl.ft, pl.fy
    tape = max(4, int(tape))
    # ---- buffers: inputs [pi][ct_y][bc][ct tallies]; results [ct_bc][scratch][ctl][stats] | [ct_pi][trunc] | [tape]
    i_pi = list(range(nP))
    i_cty = list(range(nP, nP + len(fy)))
    i_bc = list(range(nP + len(fy), nP + len(fy) + nB))
    i_ctt = list(range(nP + len(fy) + nB, nP + len(fy) + nB + len(ft)))
    n_in = nP + len(fy) + nB + len(ft)
    res = []

    def result(shape, dt, per_item=False):
        res.append((tuple(shape), np.dtype(dt), per_item))
        return n_in + len(res) - 1
    r_gbc = {j: result(bav[j].shape, np.float32) for j in adj.wrt_bc}
    r_scr = {j: result((K.exact_words(max(1, bav[j].size)),), np.uint32) for j in adj.wrt_bc}
    r_ctl = result((8,), np.uint32)
    r_stats = result((5,), np.int32)
    n_zero = len(res)
    r_gpi = {i: result(pav[i].shape, np.float32, per_item=True) for i in adj.wrt_pi}
    r_tr = result((), np.bool_, per_item=True) if prog.trunc is not None else None
    pre_act_in, P_act, car_act, bconst_act = pl.pre_act_in, pl.P_act, pl.car_act, pl.bconst_act
    if not any(car_act):
        raise ReverseError("internal: the step-scheduled adjoint is for programs with an active loop carry")

    def ct_read(slot, idx):
        if slot not in ft:
            return np.float32(0.0)
        return C.bind("tm_ct_read", [idx.var if C.is_traced(idx) else C.literal(int(idx), C.I32, False)],
                      [C.AVal((), C.F32)], slot=slot)[0]
    nbc = len(sp.bconst)
    body_slots = {nbc + j: s for j, s in enumerate(sp.car_slot) if s is not None}
    fused, f_ctout, f_ctin = AD.vjp_jaxpr(sp.body, bconst_act + car_act, ct_read, body_slots, ct_given=car_act,
                                         with_primal=True)
    post_slots = {sp.nP + j: s for j, s in enumerate(sp.car_slot) if s is not None}
    post_vjp, p_ctout, p_ctin = AD.vjp_jaxpr(sp.post, P_act + list(car_act), ct_read, post_slots)
    pre_vjp, r_ctout, r_ctin = AD.vjp_jaxpr(sp.pre, pre_act_in, ct_read, {k: k for k in range(nT)})
    for ci, ca in zip(f_ctin[nbc:], car_act):
        if ci and not ca:
            raise ReverseError("internal: carry activity mismatch")

    em = Emitter()
    em.hooks["tallymap_emit"] = lambda em_, e, ins: ins[0]

    def ct_rule(em_, e, ins):
        k = e.params["slot"]
        S = prog.tallies[k].S
        idx = ins[0].el[0]
        ptr = f"((const float*)P.p[{i_ctt[ft.index(k)]}])"
        return Val([em_.bind(f"((u32)({idx}) < {S}u ? {ptr}[{idx}] : 0.0f)", C.F32, "ct")], (), C.F32)
    em.hooks["tm_ct_read"] = ct_rule
    lines = []

    def out(s, ind=0):
        lines.append("  " * ind + s)

    def run_block(jxp, ins, ind):
        em.lines, em.ind = [], ind
        r = em.run(jxp, ins)
        lines.extend(em.lines)
        return r

    # ---- per-lane state (kernel scope): carries, lambda, loop-constant cotangents, P values, per-item operands
    decls = []

    def declare(dt, name):
        decls.append(f"  {ctype(dt)} {name};")
        return name
    bvals = [Val([f"tm_b{i}_{e}" for e in range(max(1, a.size))], a.shape, a.dtype) for i, a in enumerate(bav)]
    tallies = [VTally(k) for k in range(nT)]
    car_avals = [v.aval for v in sp.body.outvars]
    car_names = []
    for j, a in enumerate(car_avals):
        if sp.car_slot[j] is not None:
            car_names.append(None)
        else:
            car_names.append([declare(a.dtype, f"tm_c{j}_{e}") for e in range(max(1, a.size))])

    def car_vals(names=None):
        names = names or car_names
        return [VTally(sp.car_slot[j]) if nm is None else Val(nm, car_avals[j].shape, car_avals[j].dtype)
                for j, nm in enumerate(names)]
    st = [(n, car_avals[j].dtype) for j, nm in enumerate(car_names) if nm is not None for n in nm]
    W = sum(_nwords(dt) for _, dt in st)
    Wp = W if W <= 2 else -(-W // 4) * 4      # (a lane's tape slot: whole 16-byte units)
    lam = {j: [declare(np.float32, f"tm_l{j}_{e}") for e in range(len(car_names[j]))]
           for j in range(len(car_names)) if car_names[j] is not None and car_act[j]}
    gq = [q for q in range(nbc) if f_ctin[q]]
    gk = {q: [declare(np.float32, f"tm_gk{q}_{e}") for e in range(max(1, sp.body.invars[q].aval.size))] for q in gq}
    P_avals = [v.aval for v in sp.pre.outvars[sp.ncar:]]
    P_names = [[declare(a.dtype, f"tm_p{q}_{e}") for e in range(max(1, a.size))] for q, a in enumerate(P_avals)]
    Pv = [Val(nm, a.shape, a.dtype) for nm, a in zip(P_names, P_avals)]
    pi_names = [[declare(a.dtype, f"tm_x{i}_{e}") for e in range(max(1, a.size))] for i, a in enumerate(pav)]
    pis = [Val(nm, a.shape, a.dtype) for nm, a in zip(pi_names, pav)]

    def const_val(ref):
        kind, x = ref
        return em.value_of({}, x) if kind == "L" else Pv[x]
    cc_vals = [const_val(r) for r in sp.cconst]
    bc_vals = [const_val(r) for r in sp.bconst]

    # ---- tape access: lane-major, word w of slot k of lane l at (l * tape + k) * Wp + w.  Step refill puts a
    # wave's lanes at different steps, so a slot-major layout (word w of slot k of every lane side by side) made
    # each 4-byte access its own line; here a lane's state is Wp contiguous words (W padded to a multiple of 4:
    # whole 16-byte units) and its consecutive steps fill consecutive ones, which L2 combines into whole lines.
    def tape_addr(slot, w):
        return f"tm_tape[(tm_lg * {tape}ull + (u64)({slot})) * {Wp}u + {w}u]"

    def tape_store(slot, names_dts, ind):
        w = 0
        for n, dt in names_dts:
            if _nwords(dt) == 2:
                out(f"{{ const u64 b = __builtin_bit_cast(u64, {n}); {tape_addr(slot, w)} = (u32)b; "
                    f"{tape_addr(slot, w + 1)} = (u32)(b >> 32); }}", ind)
                w += 2
            elif ctype(dt) == "bool":
                out(f"{tape_addr(slot, w)} = (u32){n};", ind)
                w += 1
            elif ctype(dt) in ("float", "u32", "i32"):
                out(f"{tape_addr(slot, w)} = __builtin_bit_cast(u32, {n});", ind)
                w += 1
            else:
                out(f"{tape_addr(slot, w)} = (u32){n};", ind)
                w += 1

    def tape_load(slot, names_dts, ind):
        w = 0
        for n, dt in names_dts:
            ct = ctype(dt)
            if _nwords(dt) == 2:
                out(f"{n} = __builtin_bit_cast({ct}, (u64){tape_addr(slot, w)} | ((u64){tape_addr(slot, w + 1)} << 32));",
                    ind)
                w += 2
            elif ct == "bool":
                out(f"{n} = {tape_addr(slot, w)} != 0u;", ind)
                w += 1
            elif ct in ("float", "u32", "i32"):
                out(f"{n} = __builtin_bit_cast({ct}, {tape_addr(slot, w)});", ind)
                w += 1
            else:
                out(f"{n} = ({ct}){tape_addr(slot, w)};", ind)
                w += 1

    def body_fwd(ind):
        em.lines, em.ind = [], ind
        cars = car_vals()
        o = em.run(sp.body, bc_vals + cars)
        assign_carries(em, cars, o)
        lines.extend(em.lines)

    def cond_pred(ind):
        return run_block(sp.cond, cc_vals + car_vals(), ind)[0].el[0]

    # input temporaries of the fused step (the state it differentiates at) and of its lambda
    in_names = [None if nm is None else [declare(car_avals[j].dtype, f"tm_i{j}_{e}") for e in range(len(nm))]
                for j, nm in enumerate(car_names)]
    st_in = [(n, car_avals[j].dtype) for j, nm in enumerate(in_names) if nm is not None for n in nm]
    lin = {j: [declare(np.float32, f"tm_li{j}_{e}") for e in range(len(v))] for j, v in lam.items()}

    def fused_step(ind, keep_primal, rev_cond):
        """the fused program at the state in tm_i* with lambda tm_li*; keep_primal: a C condition under which the
        primal outputs become the carries; rev_cond: under which lambda and the constants' cotangents update."""
        cts = []
        for j, m in enumerate(f_ctout):
            if m:
                cts.append(Val(lin[j], car_avals[j].shape, C.F32) if j in lin
                           else Val(["0.0f"] * max(1, car_avals[j].size), car_avals[j].shape, C.F32))
        r = run_block(fused, bc_vals + car_vals(in_names) + cts, ind)
        prim, grads = r[:len(sp.body.outvars)], r[len(sp.body.outvars):]
        if keep_primal:
            out(f"if ({keep_primal}) {{", ind)
            for j, nm in enumerate(car_names):
                if nm is not None:
                    for n, el in zip(nm, prim[j].el):
                        out(f"{n} = {el};", ind + 1)
            out("}", ind)
        out(f"if ({rev_cond}) {{", ind)
        k = 0
        for q, m in enumerate(f_ctin):
            if not m:
                continue
            v = grads[k]
            k += 1
            if q < nbc:
                for n, el in zip(gk[q], v.el):
                    out(f"{n} = {n} + {el};", ind + 1)
            elif (q - nbc) in lam:
                for n, el in zip(lam[q - nbc], v.el):
                    out(f"{n} = {el};", ind + 1)
        out("}", ind)

    # ---------------------------------------------------------------------------------------------- source
    from . import compile as Cm
    R = n_in + len(res) + 1
    r_tape = n_in + len(res)
    res.append(((tape * Wp,), np.dtype(np.uint32), "tape"))
    src = [Cm.prelude(), f"struct TmParams {{ void* p[{R}]; }};",
           f"#define TM_STATS ((i32*)P.p[{r_stats}])", f"#define TM_CTL ((u32*)P.p[{r_ctl}])"]
    zero_words = []
    for j in adj.wrt_bc:
        zero_words.append((r_gbc[j], max(1, bav[j].size)))
        zero_words.append((r_scr[j], K.exact_words(max(1, bav[j].size))))
    zero_words += [(r_ctl, 8), (r_stats, 5)]
    src.append("extern \"C\" __global__ void tm_zero(const TmParams P, const i64 n_items) {\n"
               "  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, s = (i64)gridDim.x * blockDim.x;\n"
               + "\n".join(f"  for (i64 i = g; i < {nw}; i += s) ((u32*)P.p[{b}])[i] = 0u;" for b, nw in zero_words)
               + "\n}")
    post_l = []
    for j in adj.wrt_bc:
        S = max(1, bav[j].size)
        words = f"((const u64*)P.p[{r_scr[j]}])"
        fl = f"((const u32*)P.p[{r_scr[j]}] + {2 * K.XW * S})"
        post_l.append(f"for (i64 i = g; i < {S}; i += st) {{ bool bad = false; "
                      f"const float o = tm_xread(&{words}[i * {K.XW}], &bad); "
                      f"const bool f = (({fl}[i >> 5] >> (i & 31)) & 1u) != 0u; "
                      f"if (f || bad) atomicAdd(&TM_STATS[3], 1); "
                      f"((float*)P.p[{r_gbc[j]}])[i] = (TM_CTL[2] != 0u || f || bad) ? __builtin_nanf(\"\") : o; }}")
    for i in adj.wrt_pi:
        n = max(1, pav[i].size)
        post_l.append(f"if (TM_CTL[2] != 0u) for (i64 i = g; i < n_items * {n}; i += st) "
                      f"((float*)P.p[{r_gpi[i]}])[i] = __builtin_nanf(\"\");")
    src.append("extern \"C\" __global__ void tm_post(const TmParams P, const i64 n_items) {\n"
               "  const i64 g = (i64)blockIdx.x * blockDim.x + threadIdx.x, st = (i64)gridDim.x * blockDim.x;\n  "
               + "\n  ".join(post_l) + "\n}")

    out(f"extern \"C\" __global__ void __launch_bounds__({block}) tm_adjoint(const TmParams P, const i64 n_items) {{")
    out(f"  u64* const tm_ctr = (u64*)P.p[{r_ctl}];")
    for j in adj.wrt_bc:
        S = max(1, bav[j].size)
        out(f"  __shared__ u64 tm_xsh{j}[{K.XW * S}];")
        out(f"  __shared__ u32 tm_xfl{j}[{(S + 31) // 32}];")
        out(f"  for (int i = threadIdx.x; i < {K.XW * S}; i += blockDim.x) tm_xsh{j}[i] = 0ull;")
        out(f"  for (int i = threadIdx.x; i < {(S + 31) // 32}; i += blockDim.x) tm_xfl{j}[i] = 0u;")
    if adj.wrt_bc:
        out("  __syncthreads();")
    for i, a in enumerate(bav):
        for e in range(max(1, a.size)):
            out(f"  const {ctype(a.dtype)} tm_b{i}_{e} = ((const {ctype(a.dtype)}*)P.p[{i_bc[i]}])[{e}];")
    out(f"  u32* const tm_tape = (u32*)P.p[{r_tape}];")
    out("  const u64 tm_lg = (u64)blockIdx.x * blockDim.x + threadIdx.x, tm_nl = (u64)gridDim.x * blockDim.x;")
    out("  u32 tm_ntr = 0;")
    out("  i32 tm_ph = 0, tm_K = 0, tm_j = 0;      // phase: 0 free, 1 counting, 2 reversing")
    out("  bool tm_fin = false, tm_more = true;")
    out("  i64 tm_item = 0;")
    out("  u64 tm_cur = 0, tm_end = 0;")
    lines.extend(decls)
    out("  while (true) {")
    # ---- claim: the wave's chunk; free lanes take items by rank
    out("    if (tm_more) {")
    out("      const u64 tm_need = tm_ballot(tm_ph == 0);")
    if refill > 1:
        out(f"      if (tm_need != 0ull && (__builtin_popcountll(tm_need) >= {int(refill)} || "
            "tm_ballot(tm_ph != 0) == 0ull)) {")
    else:
        out("      if (tm_need != 0ull) {")
    out("        if (tm_cur >= tm_end) {")
    out(f"          const u64 tm_b = tm_claim(tm_ctr, {chunk}u);")
    out("          if (tm_b >= (u64)n_items) {")
    out("            tm_more = false;")
    out("          } else {")
    out(f"            tm_cur = tm_b; tm_end = tm_b + {chunk}u < (u64)n_items ? tm_b + {chunk}u : (u64)n_items;")
    out("          }")
    out("        }")
    out("        if (tm_cur < tm_end) {")
    out("          const u64 tm_av = tm_end - tm_cur;")
    out("          const u64 tm_n = (u64)__builtin_popcountll(tm_need);")
    out("          if (tm_ph == 0) {")
    out("            const u64 tm_r = tm_rank(tm_need);")
    out("            if (tm_r < tm_av) {")
    out("              tm_item = (i64)(tm_cur + tm_r);")
    # operands -> state; PRE -> carries, P values; K = 0; constants' cotangents = 0
    for i, a in enumerate(pav):
        n = max(1, a.size)
        for e in range(n):
            out(f"{pi_names[i][e]} = ((const {ctype(a.dtype)}*)P.p[{i_pi[i]}])[tm_item * {n} + {e}];", 7)
    pre_outs = run_block(sp.pre, tallies + pis + bvals, 7)
    for j, nm in enumerate(car_names):
        if nm is not None:
            for n, el in zip(nm, pre_outs[j].el):
                out(f"{n} = {el};", 7)
    for q, nm in enumerate(P_names):
        for n, el in zip(nm, pre_outs[sp.ncar + q].el):
            out(f"{n} = {el};", 7)
    for q in gq:
        for n in gk[q]:
            out(f"{n} = 0.0f;", 7)
    out("tm_K = 0;", 7)
    out("tm_ph = 1;", 7)
    out("            }")
    out("          }")
    out("          tm_cur += tm_n < tm_av ? tm_n : tm_av;")
    out("          if (tm_cur >= tm_end && tm_end >= (u64)n_items) tm_more = false;")
    out("        }")
    out("      }")
    out("    }")
    # ---- counting lanes whose loop ended: POST, POST's VJP, then reverse (or the long-item sweep)
    out("    if (tm_ph == 1) {")
    p = cond_pred(3)
    out(f"      if (!({p})) {{")
    post_ins = Pv + car_vals()
    post_fwd = run_block(sp.post, post_ins, 4)
    if prog.trunc is not None:
        tr = post_fwd[nT + prog.trunc].el[0]
        out(f"((bool*)P.p[{r_tr}])[tm_item] = {tr};", 4)
        out(f"if ({tr}) ++tm_ntr;", 4)
    post_cts = []
    for j, (o, m) in enumerate(zip(sp.post.outvars, p_ctout)):
        if not m:
            continue
        q = j - nT
        if q >= 0 and q in fy:
            a = yav[q]
            n = max(1, a.size)
            post_cts.append(Val([f"((const float*)P.p[{i_cty[fy.index(q)]}])[tm_item * {n} + {e}]" for e in range(n)],
                                a.shape, C.F32))
        else:
            post_cts.append(Val(["0.0f"] * max(1, o.aval.size), o.aval.shape, C.F32))
    pr = run_block(post_vjp, post_ins + post_cts, 4)
    gP = {}
    k = 0
    for q, m in enumerate(p_ctin):
        if not m:
            continue
        v = pr[k]
        k += 1
        if q < sp.nP:
            gP[q] = [declare(np.float32, f"tm_gp{q}_{e}") for e in range(len(v.el))]
            for n, el in zip(gP[q], v.el):
                out(f"{n} = {el};", 4)
        elif (q - sp.nP) in lam:
            for n, el in zip(lam[q - sp.nP], v.el):
                out(f"{n} = {el};", 4)
    for j, names in lam.items():
        if not p_ctin[sp.nP + j]:
            for n in names:
                out(f"{n} = 0.0f;", 4)
    out(f"if (tm_K <= {tape}) {{", 4)
    out("tm_j = tm_K - 1;", 5)
    out("tm_ph = 2;", 5)
    out("if (tm_j < 0) tm_fin = true;", 5)
    out("} else {", 4)
    # the long item: checkpoints every m steps in slots [0, H), each segment's states in [H, tape)
    H = tape // 2
    Sg = tape - H
    out(f"const i32 tm_m = (tm_K + {H - 1}) / {H};", 5)
    tape_load("0", st, 5)
    out("for (i32 tm_k = 0; tm_k < tm_K; ++tm_k) {", 5)
    out("if (tm_k % tm_m == 0) {", 6)
    tape_store("tm_k / tm_m", st, 7)
    out("}", 6)
    body_fwd(6)
    out("}", 5)
    out("const i32 tm_ns = (tm_K + tm_m - 1) / tm_m;", 5)
    out("for (i32 tm_s = tm_ns - 1; tm_s >= 0; --tm_s) {", 5)
    out("const i32 tm_a = tm_s * tm_m, tm_bb = tm_a + tm_m < tm_K ? tm_a + tm_m : tm_K;", 6)
    out("for (i32 tm_hi = tm_bb; tm_hi > tm_a;) {", 6)
    out(f"const i32 tm_lo = tm_hi - {Sg} > tm_a ? tm_hi - {Sg} : tm_a;", 7)
    tape_load("tm_s", st, 7)
    out("for (i32 tm_k = tm_a; tm_k < tm_lo; ++tm_k) {", 7)
    body_fwd(8)
    out("}", 7)
    out("for (i32 tm_k = tm_lo; tm_k < tm_hi; ++tm_k) {", 7)
    tape_store(f"{H} + tm_k - tm_lo", st, 8)
    body_fwd(8)
    out("}", 7)
    out("for (i32 tm_k = tm_hi - 1; tm_k >= tm_lo; --tm_k) {", 7)
    tape_load(f"{H} + tm_k - tm_lo", st_in, 8)
    for j, names in lin.items():
        for a_, b_ in zip(names, lam[j]):
            out(f"{a_} = {b_};", 8)
    fused_step(8, None, "true")
    out("}", 7)
    out("tm_hi = tm_lo;", 7)
    out("}", 6)
    out("}", 5)
    out("tm_fin = true;", 5)
    out("}", 4)
    out("      }")
    out("    }")
    # ---- one step of every counting or reversing lane
    out("    if (tm_ph != 0 && !tm_fin) {")
    out("      if (tm_ballot(tm_ph == 2) != 0ull) {")
    for (a_, dt), (b_, _) in zip(st_in, st):
        out(f"{a_} = {b_};", 4)
    out("if (tm_ph == 2) {", 4)
    tape_load("tm_j", st_in, 5)
    out("}", 4)
    for j, names in lin.items():
        for a_, b_ in zip(names, lam[j]):
            out(f"{a_} = tm_ph == 2 ? {b_} : 0.0f;", 4)
    out(f"if (tm_ph == 1 && tm_K < {tape}) {{", 4)
    tape_store("tm_K", st, 5)
    out("}", 4)
    fused_step(4, "tm_ph == 1", "tm_ph == 2")
    out("if (tm_ph == 1) {", 4)
    out("++tm_K;", 5)
    out("} else {", 4)
    out("--tm_j;", 5)
    out("if (tm_j < 0) tm_fin = true;", 5)
    out("}", 4)
    out("      } else {")
    out(f"if (tm_K < {tape}) {{", 4)
    tape_store("tm_K", st, 5)
    out("}", 4)
    body_fwd(4)
    out("++tm_K;", 4)
    out("      }")
    out("    }")
    # ---- finish: PRE's VJP
    out("    if (tm_fin) {")
    pre_cts = []
    for j, (o, m) in enumerate(zip(sp.pre.outvars, r_ctout)):
        if not m:
            continue
        if j < sp.ncar:
            pre_cts.append(Val(lam[j], o.aval.shape, C.F32) if j in lam
                           else Val(["0.0f"] * max(1, o.aval.size), o.aval.shape, C.F32))
        else:
            q = j - sp.ncar
            terms = [gP[q]] if q in gP else []
            for bq, r in enumerate(sp.bconst):
                if r[0] == "P" and r[1] == q and bq in gk:
                    terms.append(gk[bq])
            n = max(1, o.aval.size)
            if not terms:
                pre_cts.append(Val(["0.0f"] * n, o.aval.shape, C.F32))
            else:
                el = []
                for e in range(n):
                    ex = terms[0][e]
                    for t in terms[1:]:
                        ex = f"({ex} + {t[e]})"
                    el.append(ex)
                pre_cts.append(Val(el, o.aval.shape, C.F32))
    gr = run_block(pre_vjp, tallies + pis + bvals + pre_cts, 3)
    k = 0
    for q, m in enumerate(r_ctin):
        if not m:
            continue
        v = gr[k]
        k += 1
        if nT <= q < nT + nP:
            i = q - nT
            n = max(1, pav[i].size)
            for e, el in enumerate(v.el):
                out(f"((float*)P.p[{r_gpi[i]}])[tm_item * {n} + {e}] = {el};", 3)
        elif q >= nT + nP:
            jb = q - nT - nP
            for e, el in enumerate(v.el):
                out(f"if (tm_xemit(&tm_xsh{jb}[{e * K.XW}], {el})) atomicOr(&tm_xfl{jb}[{e >> 5}], "
                    f"{1 << (e & 31)}u);", 3)
    for i in adj.wrt_pi:
        if not r_ctin[nT + i]:
            n = max(1, pav[i].size)
            for e in range(n):
                out(f"((float*)P.p[{r_gpi[i]}])[tm_item * {n} + {e}] = 0.0f;", 3)
    out("      tm_fin = false;")
    out("      tm_ph = 0;")
    out("    }")
    out("    if (tm_ballot(tm_ph != 0 || tm_more) == 0ull) break;")
    out("  }")
    out("  if (tm_ntr) atomicAdd(&TM_CTL[2], tm_ntr);")
    if adj.wrt_bc:
        out("  __syncthreads();")
        for j in adj.wrt_bc:
            S = max(1, bav[j].size)
            gw = f"((u64*)P.p[{r_scr[j]}])"
            gf = f"((u32*)P.p[{r_scr[j]}] + {2 * K.XW * S})"
            out(f"  for (int i = threadIdx.x; i < {K.XW * S}; i += blockDim.x) {{ const i64 x = (i64)tm_xsh{j}[i]; "
                f"if (x != 0 && tm_xadd(&{gw}[i / {K.XW} * {K.XW}], i % {K.XW}, x)) "
                f"atomicOr(&{gf}[(i / {K.XW}) >> 5], 1u << ((i / {K.XW}) & 31)); }}")
            out(f"  for (int i = threadIdx.x; i < {(S + 31) // 32}; i += blockDim.x) "
                f"if (tm_xfl{j}[i]) atomicOr(&{gf}[i], tm_xfl{j}[i]);")
    out("}")
    # the declarations gathered while emitting (POST's P cotangents) go to the kernel scope too
    body = "\n".join(lines)
    marker = "  u64 tm_cur = 0, tm_end = 0;"
    body = body.replace(marker, marker + "\n" + "\n".join(d for d in decls if d not in lines), 1)
    src.append(body)
    L = K.Layout(n_in=n_in, res=res, n_zero=n_zero, r_out=r_gbc, r_ctl=r_ctl, r_stats=r_stats,
                 r_ys=[r_gpi[i] for i in adj.wrt_pi] + ([r_tr] if r_tr is not None else []), flags=2,
                 mode="adjoint-step", priv=list(adj.wrt_bc), zero_words=zero_words)
    L.i_pi, L.i_cty, L.i_bc, L.i_ctt, L.ft, L.fy = i_pi, i_cty, i_bc, i_ctt, ft, fy
    return "\n\n".join(src), L


def tape_bytes(layout, lanes):
    """bytes of the tape buffer for `lanes` launched lanes."""
    for shape, dt, kind in layout.res:
        if kind == "tape":
            return int(np.prod(shape)) * np.dtype(dt).itemsize * int(lanes)
    return 0


