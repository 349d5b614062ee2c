// Config-3 form at a small size: bf16 x, bf16 weight stored [N, K] and used
// transposed, bf16 bias; nova.linear in f32 after widening casts, GELU, and
// a cast of the result back to bf16.
module {
  func.func @linear_gelu(%x: tensor<96x160xbf16>, %w: tensor<200x160xbf16>, %b: tensor<200xbf16>) -> tensor<96x200xbf16> {
    %xf = nova.cast %x : tensor<96x160xbf16> -> tensor<96x160xf32>
    %wt = nova.transpose %w : tensor<200x160xbf16>
    %wf = nova.cast %wt : tensor<160x200xbf16> -> tensor<160x200xf32>
    %bf = nova.cast %b : tensor<200xbf16> -> tensor<200xf32>
    %y = nova.linear %xf, %wf, %bf : tensor<96x160xf32>, tensor<160x200xf32>, tensor<200xf32>
    %g = nova.gelu %y : tensor<96x200xf32>
    %o = nova.cast %g : tensor<96x200xf32> -> tensor<96x200xbf16>
    return %o : tensor<96x200xbf16>
  }
}
