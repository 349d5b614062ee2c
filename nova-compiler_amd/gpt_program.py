"""A GPT training step in the Nova op surface, as text, for any sizes: token
and position embeddings (nova.gather), LayerNorm, an MLP block with GELU and
a residual add, a final LayerNorm, the LM-head matmul, the SCE loss and the
whole backward pass down to the embedding gradients (nova.scatter_add).  It
uses the ops of the reference's GPT step (ltest/test.mlir): the operation
sequence has to be alike to exercise the same ops.  Unlike that file it
passes the forward's saved statistics to nova.layer_norm_backward (the op's
five operands, NovaOps.td:1041-1042) and the softmax, not the logits, to
nova.sce_backward (NovaToLinalgGeneric.cpp:1031, "Softmax is passed in
directly").  Results are returned instead of added into writable memref
arguments."""


def gpt_step(B, T, V, D, H):
    N = B * T
    t = lambda *s: "tensor<" + "x".join(str(x) for x in s) + ">"  # noqa: E731
    f = lambda *s: t(*s, "f32")  # noqa: E731
    args = [("tok", t(B, T, "i16")), ("tgt", t(B, T, "i16")), ("pos", t(1, T, "i64")),
            ("wte", f(V, D)), ("wpe", f(T, D)), ("g1", f(D)), ("be1", f(D)),
            ("w1", f(D, H)), ("c1", f(H)), ("w2", f(H, D)), ("c2", f(D)),
            ("g2", f(D)), ("be2", f(D)), ("wlm", f(D, V))]
    rets = [("%sce#1", f(1)), ("%dwte", f(V, D)), ("%dwpe", f(T, D)), ("%gh#1", f(D)),
            ("%gh#2", f(D)), ("%gu#1", f(D, H)), ("%gu#2", f(H)), ("%gd#1", f(H, D)),
            ("%gd#2", f(D)), ("%gr#1", f(D)), ("%gr#2", f(D)), ("%dwlm", f(D, V))]
    x3, h3 = f(B, T, D), f(B, T, H)
    body = f"""
  %x_tok = nova.gather %wte [%tok] : {f(V, D)}, {t(B, T, 'i16')} -> {x3}
  %x_pos = nova.gather %wpe [%pos] : {f(T, D)}, {t(1, T, 'i64')} -> {f(1, T, D)}
  %h = nova.add %x_tok, %x_pos : {x3}, {f(1, T, D)}
  %ln1:3 = nova.layer_norm %h, %g1, %be1 : {x3}, {f(D)}, {f(D)}
  %up = nova.linear %ln1#0, %w1, %c1 : {x3}, {f(D, H)}, {f(H)}
  %act = nova.gelu %up : {h3}
  %dn = nova.linear %act, %w2, %c2 : {h3}, {f(H, D)}, {f(D)}
  %r = nova.add %h, %dn : {x3}, {x3}
  %ln2:3 = nova.layer_norm %r, %g2, %be2 : {x3}, {f(D)}, {f(D)}
  %flat = nova.reshape %ln2#0 : {x3} -> {f(N, D)}
  %lg = nova.matmul %flat, %wlm : {f(N, D)}, {f(D, V)}
  %logits = nova.reshape %lg : {f(N, V)} -> {f(B, T, V)}
  %sce:2 = nova.sce %logits, %tgt : {f(B, T, V)}, {t(B, T, 'i16')}
  %one = nova.constant {{value = dense<1.000000e+00> : {f(1)}}} : {f(1)}
  %dl0 = nova.sce_backward %sce#0, %tgt : {f(B, T, V)}, {t(B, T, 'i16')}
  %dl = nova.mul %dl0, %one : {f(B, T, V)}, {f(1)}
  %dlf = nova.reshape %dl : {f(B, T, V)} -> {f(N, V)}
  %flat_t = nova.transpose %flat : {f(N, D)}
  %wlm_t = nova.transpose %wlm : {f(D, V)}
  %dflat = nova.matmul %dlf, %wlm_t : {f(N, V)}, {f(V, D)}
  %dwlm = nova.matmul %flat_t, %dlf : {f(D, N)}, {f(N, V)}
  %dln2 = nova.reshape %dflat : {f(N, D)} -> {x3}
  %gr:3 = nova.layer_norm_backward %dln2, %r, %g2, %ln2#1, %ln2#2 : {x3}, {x3}, {f(D)}, {f(B, T)}, {f(B, T)}
  %gd:3 = nova.linear_backward %gr#0, %act, %w2 : {x3}, {h3}, {f(H, D)}
  %dup = nova.gelu_backward %gd#0, %up : {h3}, {h3}
  %gu:3 = nova.linear_backward %dup, %ln1#0, %w1 : {h3}, {x3}, {f(D, H)}
  %gh:3 = nova.layer_norm_backward %gu#0, %h, %g1, %ln1#1, %ln1#2 : {x3}, {x3}, {f(D)}, {f(B, T)}, {f(B, T)}
  %dh = nova.add %gr#0, %gh#0 : {x3}, {x3}
  %dpos = nova.reduce<sum> %dh dimension = [0] : {x3}
  %pos1 = nova.reshape %pos : {t(1, T, 'i64')} -> {t(T, 'i64')}
  %zpos = nova.constant {{value = dense<0.000000e+00> : {f(T, D)}}} : {f(T, D)}
  %dwpe = nova.scatter_add %zpos, %pos1, %dpos : {f(T, D)}, {t(T, 'i64')}, {f(T, D)} -> {f(T, D)}
  %tok1 = nova.reshape %tok : {t(B, T, 'i16')} -> {t(N, 'i16')}
  %dh2 = nova.reshape %dh : {x3} -> {f(N, D)}
  %zte = nova.constant {{value = dense<0.000000e+00> : {f(V, D)}}} : {f(V, D)}
  %dwte = nova.scatter_add %zte, %tok1, %dh2 : {f(V, D)}, {t(N, 'i16')}, {f(N, D)} -> {f(V, D)}
  return {", ".join(r for r, _ in rets)} : {", ".join(ty for _, ty in rets)}
"""
    sig = ", ".join(f"%{n}: {ty}" for n, ty in args)
    res = ", ".join(ty for _, ty in rets)
    return f"func.func @gpt_step({sig}) -> ({res}) {{{body}}}\n"
