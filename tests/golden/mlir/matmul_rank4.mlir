// nova.matmul above rank 3 (the reference collapses the batch dims to one
// and expands them back, NovaToLinalg.cpp:904-988), with a rank-2 operand
// broadcast over them; and a transpose of batch axes feeding the product,
// whose permuted leading dims the launch cannot fold (refused), as are
// labels given as a transposed view.
module {
  func.func @mm4(%A: tensor<2x3x8x16xf32>, %B: tensor<2x3x16x5xf32>) -> tensor<2x3x8x5xf32> {
    %r = nova.matmul %A, %B : tensor<2x3x8x16xf32>, tensor<2x3x16x5xf32>
    return %r : tensor<2x3x8x5xf32>
  }
  func.func @mm4_bcast(%A: tensor<2x3x8x16xf32>, %B: tensor<16x5xf32>) -> tensor<2x3x8x5xf32> {
    %r = nova.matmul %A, %B : tensor<2x3x8x16xf32>, tensor<16x5xf32>
    return %r : tensor<2x3x8x5xf32>
  }
  func.func @mm4_batch_transposed(%A: tensor<3x2x8x16xf32>, %B: tensor<2x3x16x5xf32>) -> tensor<2x3x8x5xf32> {
    %t = nova.transpose %A {axes1 = 0 : i64, axes2 = 1 : i64} : tensor<3x2x8x16xf32>
    %r = nova.matmul %t, %B : tensor<2x3x8x16xf32>, tensor<2x3x16x5xf32>
    return %r : tensor<2x3x8x5xf32>
  }
  func.func @sce_labels_transposed(%X: tensor<8x32xf32>, %L: tensor<4x2xi32>) -> tensor<1xf32> {
    %lt = nova.transpose %L : tensor<4x2xi32>
    %x = nova.reshape %X : tensor<8x32xf32> -> tensor<2x4x32xf32>
    %s:2 = nova.sce %x, %lt : tensor<2x4x32xf32>, tensor<2x4xi32>
    return %s#1 : tensor<1xf32>
  }
}
