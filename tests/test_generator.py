"""CPU tier: the checks of the 64-row kernel generator (gen_prefill_w64.py).

The generated bodies (bf16, fp16 and MXFP8, causal and not) pass the hazard,
memory-counter, SCC and schedule checks the generator runs before writing
them; and each check rejects a planted mistake of the kind it exists for: a
dropped LDS wait, an MFMA result read too early, an SCC reader behind a
foreign SCC writer, a schedule that reorders a dependent pair.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "cuda_amd", "csrc"))

import gen_prefill_w64 as G  # noqa: E402


@pytest.fixture(params=["bf16", "f16", "mx"])
def mode(request):
    G.configure(request.param == "mx")
    G.configure_f16(request.param == "f16")
    yield request.param
    G.configure_f16(False)
    G.configure(False)


def _prog(causal):
    g = G.Gen(causal)
    return g, g.kernel()


def _steady_start(prog, tag):
    return next(i for i, x in enumerate(prog) if x.kind == "label" and x.text == f"L_pfw64{tag}_steady1:")


@pytest.mark.parametrize("causal", [True, False])
def test_generated_bodies_pass_checks(mode, causal):
    g, prog = _prog(causal)
    assert G.check(prog, g.tag)
    G.check_scc(prog, g.tag)
    kinds = {x.kind for x in prog}
    assert {"mfma", "lds", "vmem", "valu", "salu", "barrier", "wait"} <= kinds
    scale = [x for x in prog if x.kind == "mfma" and "scale" in x.text]
    assert bool(scale) == (mode == "mx")    # the MX body runs QK on the scaled fp8 MFMA
    f16 = [x for x in prog if x.kind == "mfma" and "_f16 " in x.text]
    assert bool(f16) == (mode == "f16")     # only the fp16 body runs the fp16 MFMA


def test_dropped_lds_wait_is_rejected(mode):
    """The first steady iteration's wait for its prefetched fragments (the
    lgkmcnt before its first MFMA) is what makes the fragment registers
    readable: without it the counter check fails."""
    g, prog = _prog(True)
    i0 = _steady_start(prog, g.tag)
    w = next(i for i in range(i0, len(prog)) if prog[i].kind == "wait" and prog[i].wlgkm is not None
             and prog[i + 1].kind == "mfma")
    bad = prog[:w] + prog[w + 1:]
    with pytest.raises(G.CheckError, match="LDS operation in flight"):
        G.check(bad, g.tag)


def test_early_mfma_result_read_is_rejected(mode):
    """A VALU read of a QK accumulator right after the MFMA that writes it
    (the result needs MFMA_WS wait states)."""
    g, prog = _prog(True)
    i0 = _steady_start(prog, g.tag)
    k = next(i for i in range(i0, len(prog)) if prog[i].kind == "mfma" and ("v", 0) in prog[i].defs
             or prog[i].kind == "mfma" and ("v", 64) in prog[i].defs)
    dst = prog[k].defs[0]
    reg = G.Reg(dst[0], dst[1])
    bad = prog[:k + 1] + [G.V("v_add_f32", G.TMP[0][0], reg, reg)] + prog[k + 1:]
    with pytest.raises(G.CheckError, match="after an MFMA wrote it"):
        G.check(bad, g.tag)


def test_foreign_scc_writer_is_rejected(mode):
    """s_addc_u32 must read the carry of its own s_add_u32."""
    g, prog = _prog(False)
    k = next(i for i, x in enumerate(prog) if x.text.startswith("s_addc_u32"))
    bad = prog[:k] + [G.S("s_cmp_eq_u32", G.T[0], 0)] + prog[k:]
    with pytest.raises(AssertionError, match="reads SCC"):
        G.check_scc(bad, g.tag)


def test_reordered_dependency_is_rejected():
    """check_item_order: a reader placed before the writer it depends on."""
    x = G.v(160)
    w = G.V("v_mov_b32", x, 1)
    r = G.V("v_add_f32", G.v(161), x, x)
    items = [G.Item(w), G.Item(r, deps=[])]
    G.check_item_order(items, [w, r])
    with pytest.raises(G.CheckError, match="dataflow"):
        G.check_item_order(items, [r, w])


def test_configuration_is_reversible():
    """configure(True) or configure_f16(True), then back, gives the bf16
    body exactly (the register map and limits are rebound, not mutated)."""
    G.configure(False)
    a = G.Gen(True).kernel()
    G.configure(True)
    G.Gen(True).kernel()
    G.configure(False)
    G.configure_f16(True)
    c = G.Gen(True).kernel()
    G.configure_f16(False)
    b = G.Gen(True).kernel()
    assert [x.text for x in a] == [x.text for x in b]
    # the fp16 body is the bf16 one with the MFMA, the P packs and the redo
    # bound (2^48 for bf16 P, 2^15 for fp16 P) changed
    assert len(a) == len(c)
    ct = [y.text.replace("pfw64HC", "pfw64C") for y in c]   # labels carry the body's tag
    diff = {(x.text.split()[0], y.split()[0]) for x, y in zip(a, ct) if x.text != y}
    assert diff == {("v_mfma_f32_32x32x16_bf16", "v_mfma_f32_32x32x16_f16"),
                    ("v_cvt_pk_bf16_f32", "v_cvt_pk_f16_f32"), ("s_mov_b32", "s_mov_b32")}, diff
    bounds = [(x.text, y) for x, y in zip(a, ct) if x.text.startswith("s_mov_b32") and x.text != y]
    assert len(bounds) == 1 and "0x57800000" in bounds[0][0] and "0x47000000" in bounds[0][1]
