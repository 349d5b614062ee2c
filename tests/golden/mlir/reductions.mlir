// Config-5 forms at small sizes, forward and backward.
module {
  func.func @ln(%x: tensor<64x1024xf32>, %g: tensor<1024xf32>, %b: tensor<1024xf32>) -> (tensor<64x1024xf32>, tensor<64xf32>, tensor<64xf32>) {
    %y, %s, %r = nova.layer_norm %x, %g, %b : tensor<64x1024xf32>, tensor<1024xf32>, tensor<1024xf32>
    return %y, %s, %r : tensor<64x1024xf32>, tensor<64xf32>, tensor<64xf32>
  }
  func.func @ln_train(%x: tensor<64x1024xf32>, %g: tensor<1024xf32>, %b: tensor<1024xf32>, %gy: tensor<64x1024xf32>) -> (tensor<64x1024xf32>, tensor<64x1024xf32>, tensor<1024xf32>, tensor<1024xf32>) {
    %y:3 = nova.layer_norm %x, %g, %b : tensor<64x1024xf32>, tensor<1024xf32>, tensor<1024xf32>
    %dx, %dg, %db = nova.layer_norm_backward %gy, %x, %g, %y#1, %y#2 : tensor<64x1024xf32>, tensor<64x1024xf32>, tensor<1024xf32>, tensor<64xf32>, tensor<64xf32>
    return %y#0, %dx, %dg, %db : tensor<64x1024xf32>, tensor<64x1024xf32>, tensor<1024xf32>, tensor<1024xf32>
  }
  func.func @sce_train(%logits: tensor<32x5000xf32>, %t: tensor<32xi32>) -> (tensor<1xf32>, tensor<32x5000xf32>) {
    %sm, %loss = nova.sce %logits, %t : tensor<32x5000xf32>, tensor<32xi32>
    %g = nova.sce_backward %sm, %t {dim = -1 : i64} : tensor<32x5000xf32>, tensor<32xi32>
    return %loss, %g : tensor<1xf32>, tensor<32x5000xf32>
  }
}
