module attributes {llaccel.model = {dim = 64 : i64, n_layers = 2 : i64, n_heads = 4 : i64, n_kv_heads = 2 : i64, head_dim = 16 : i64, ffn = 176 : i64, vocab = 200 : i64, max_seq = 64 : i64, rope_base = 10000.0 : f64, rms_eps = 1e-05 : f64}} {
  llaccel.weight @embed : tensor<200x64xf32>
  llaccel.weight @l0_attn_norm : tensor<64xf32>
  llaccel.weight @l0_wq : tensor<64x64xf32>
  llaccel.weight @l0_wk : tensor<32x64xf32>
  llaccel.weight @l0_wv : tensor<32x64xf32>
  llaccel.weight @l0_wo : tensor<64x64xf32>
  llaccel.weight @l0_ffn_norm : tensor<64xf32>
  llaccel.weight @l0_wg : tensor<176x64xf32>
  llaccel.weight @l0_wu : tensor<176x64xf32>
  llaccel.weight @l0_wd : tensor<64x176xf32>
  llaccel.weight @l1_attn_norm : tensor<64xf32>
  llaccel.weight @l1_wq : tensor<64x64xf32>
  llaccel.weight @l1_wk : tensor<32x64xf32>
  llaccel.weight @l1_wv : tensor<32x64xf32>
  llaccel.weight @l1_wo : tensor<64x64xf32>
  llaccel.weight @l1_ffn_norm : tensor<64xf32>
  llaccel.weight @l1_wg : tensor<176x64xf32>
  llaccel.weight @l1_wu : tensor<176x64xf32>
  llaccel.weight @l1_wd : tensor<64x176xf32>
  llaccel.weight @norm : tensor<64xf32>
  llaccel.weight @lm_head : tensor<200x64xf32>
}
