// Matmul -> row-Softmax chain, canonical decomposed form (wtc canonicalize).
module {
  func.func @main(%A: tensor<8192x64xf16>, %B: tensor<64x128xf16>) -> tensor<8192x128xf32> {
    %acc_zero = arith.constant 0.0 : f32
    %f0 = arith.constant 0.0 : f32
    %neg_inf = arith.constant -3.4028235e+38 : f32
    %c0 = tensor.empty() : tensor<8192x128xf32>
    %c_init = linalg.fill ins(%acc_zero : f32) outs(%c0 : tensor<8192x128xf32>) -> tensor<8192x128xf32>
    %C0 = linalg.matmul
      ins(%A, %B : tensor<8192x64xf16>, tensor<64x128xf16>)
      outs(%c_init : tensor<8192x128xf32>) -> tensor<8192x128xf32>
    %x0 = tensor.empty() : tensor<8192x128xf32>
    %C = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>], iterator_types = ["parallel", "parallel"]}
      ins(%C0 : tensor<8192x128xf32>) outs(%x0 : tensor<8192x128xf32>) {
    ^bb0(%in: f32, %o: f32):
      linalg.yield %in : f32
    } -> tensor<8192x128xf32>
    %max0 = tensor.empty() : tensor<8192xf32>
    %max_init = linalg.fill ins(%neg_inf : f32) outs(%max0 : tensor<8192xf32>) -> tensor<8192xf32>
    %max = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>], iterator_types = ["parallel", "reduction"]}
      ins(%C : tensor<8192x128xf32>) outs(%max_init : tensor<8192xf32>) {
    ^bb0(%in: f32, %acc: f32):
      %m = arith.maximumf %in, %acc : f32
      linalg.yield %m : f32
    } -> tensor<8192xf32>
    %e0 = tensor.empty() : tensor<8192x128xf32>
    %exp_sub = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>, affine_map<(d0, d1) -> (d0, d1)>], iterator_types = ["parallel", "parallel"]}
      ins(%C, %max : tensor<8192x128xf32>, tensor<8192xf32>) outs(%e0 : tensor<8192x128xf32>) {
    ^bb0(%x: f32, %mx: f32, %o: f32):
      %d = arith.subf %x, %mx : f32
      %e = math.exp %d : f32
      linalg.yield %e : f32
    } -> tensor<8192x128xf32>
    %s0 = tensor.empty() : tensor<8192xf32>
    %sum_init = linalg.fill ins(%f0 : f32) outs(%s0 : tensor<8192xf32>) -> tensor<8192xf32>
    %sum = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>], iterator_types = ["parallel", "reduction"]}
      ins(%exp_sub : tensor<8192x128xf32>) outs(%sum_init : tensor<8192xf32>) {
    ^bb0(%in: f32, %acc: f32):
      %r = arith.addf %in, %acc : f32
      linalg.yield %r : f32
    } -> tensor<8192xf32>
    %y0 = tensor.empty() : tensor<8192x128xf32>
    %out = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0)>, affine_map<(d0, d1) -> (d0, d1)>], iterator_types = ["parallel", "parallel"]}
      ins(%exp_sub, %sum : tensor<8192x128xf32>, tensor<8192xf32>) outs(%y0 : tensor<8192x128xf32>) {
    ^bb0(%e: f32, %s: f32, %o: f32):
      %y = arith.divf %e, %s : f32
      linalg.yield %y : f32
    } -> tensor<8192x128xf32>
    return %out : tensor<8192x128xf32>
  }
}
