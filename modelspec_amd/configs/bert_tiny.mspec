// The BERT-tiny masked-LM config (BASELINE configs[3]): two post-layer-norm encoder layers,
// hidden 128, 2 heads, FFN 512, learned positions over 128, batches of 32, the 30,522-token
// vocabulary, the decoder tied to the token table with its own bias, dropout 0.1, AdamW 1e-4
// with a 100-step warm-up over 1,000 steps. The masked-row gather keeps 832 loss rows.
model BertTiny {
    param tok_table: Tensor<f32, [30522, 128]> = xavier_uniform();
    param pos_table: Tensor<f32, [128, 128]> = xavier_uniform();
    param emb_ln_gamma: Tensor<f32, [128]> = ones();
    param emb_ln_beta: Tensor<f32, [128]> = zeros();

    param l0_wq: Tensor<f32, [128, 128]> = xavier_uniform();
    param l0_bq: Tensor<f32, [128]> = zeros();
    param l0_wk: Tensor<f32, [128, 128]> = xavier_uniform();
    param l0_bk: Tensor<f32, [128]> = zeros();
    param l0_wv: Tensor<f32, [128, 128]> = xavier_uniform();
    param l0_bv: Tensor<f32, [128]> = zeros();
    param l0_wo: Tensor<f32, [128, 128]> = xavier_uniform();
    param l0_bo: Tensor<f32, [128]> = zeros();
    param l0_ln1_gamma: Tensor<f32, [128]> = ones();
    param l0_ln1_beta: Tensor<f32, [128]> = zeros();
    param l0_w1: Tensor<f32, [128, 512]> = xavier_uniform();
    param l0_b1: Tensor<f32, [512]> = zeros();
    param l0_w2: Tensor<f32, [512, 128]> = xavier_uniform();
    param l0_b2: Tensor<f32, [128]> = zeros();
    param l0_ln2_gamma: Tensor<f32, [128]> = ones();
    param l0_ln2_beta: Tensor<f32, [128]> = zeros();

    param l1_wq: Tensor<f32, [128, 128]> = xavier_uniform();
    param l1_bq: Tensor<f32, [128]> = zeros();
    param l1_wk: Tensor<f32, [128, 128]> = xavier_uniform();
    param l1_bk: Tensor<f32, [128]> = zeros();
    param l1_wv: Tensor<f32, [128, 128]> = xavier_uniform();
    param l1_bv: Tensor<f32, [128]> = zeros();
    param l1_wo: Tensor<f32, [128, 128]> = xavier_uniform();
    param l1_bo: Tensor<f32, [128]> = zeros();
    param l1_ln1_gamma: Tensor<f32, [128]> = ones();
    param l1_ln1_beta: Tensor<f32, [128]> = zeros();
    param l1_w1: Tensor<f32, [128, 512]> = xavier_uniform();
    param l1_b1: Tensor<f32, [512]> = zeros();
    param l1_w2: Tensor<f32, [512, 128]> = xavier_uniform();
    param l1_b2: Tensor<f32, [128]> = zeros();
    param l1_ln2_gamma: Tensor<f32, [128]> = ones();
    param l1_ln2_beta: Tensor<f32, [128]> = zeros();

    param mlm_w: Tensor<f32, [128, 128]> = xavier_uniform();
    param mlm_b: Tensor<f32, [128]> = zeros();
    param mlm_ln_gamma: Tensor<f32, [128]> = ones();
    param mlm_ln_beta: Tensor<f32, [128]> = zeros();
    param mlm_bias: Tensor<f32, [30522]> = zeros();

    fn forward(ids: Tensor<i32, [4096]>, positions: Tensor<i32, [4096]>, key_mask: Tensor<f32, [32, 128]>)
        -> Tensor<f32, [4096, 30522]> {
        let tokens = add(embedding(tok_table, ids), embedding(pos_table, positions));
        let x = dropout(layer_norm(tokens, emb_ln_gamma, emb_ln_beta), p = 0.1);

        let l0_q = add_rows(matmul(x, l0_wq), l0_bq);
        let l0_k = add_rows(matmul(x, l0_wk), l0_bk);
        let l0_v = add_rows(matmul(x, l0_wv), l0_bv);
        let l0_att = add_rows(matmul(attention(l0_q, l0_k, l0_v, key_mask, heads = 2), l0_wo), l0_bo);
        let l0_h = layer_norm(add(x, dropout(l0_att, p = 0.1)), l0_ln1_gamma, l0_ln1_beta);
        let l0_ffn = add_rows(matmul(gelu(add_rows(matmul(l0_h, l0_w1), l0_b1)), l0_w2), l0_b2);
        let l0_out = layer_norm(add(l0_h, dropout(l0_ffn, p = 0.1)), l0_ln2_gamma, l0_ln2_beta);

        let l1_q = add_rows(matmul(l0_out, l1_wq), l1_bq);
        let l1_k = add_rows(matmul(l0_out, l1_wk), l1_bk);
        let l1_v = add_rows(matmul(l0_out, l1_wv), l1_bv);
        let l1_att = add_rows(matmul(attention(l1_q, l1_k, l1_v, key_mask, heads = 2), l1_wo), l1_bo);
        let l1_h = layer_norm(add(l0_out, dropout(l1_att, p = 0.1)), l1_ln1_gamma, l1_ln1_beta);
        let l1_ffn = add_rows(matmul(gelu(add_rows(matmul(l1_h, l1_w1), l1_b1)), l1_w2), l1_b2);
        let l1_out = layer_norm(add(l1_h, dropout(l1_ffn, p = 0.1)), l1_ln2_gamma, l1_ln2_beta);

        let head = layer_norm(gelu(add_rows(matmul(l1_out, mlm_w), mlm_b)), mlm_ln_gamma, mlm_ln_beta);
        return add_rows(matmul(head, transpose(tok_table)), mlm_bias);
    }
}

train Pretrain {
    model = BertTiny;
    input ids: Tensor<i32, [4096]>;
    input positions: Tensor<i32, [4096]>;
    input key_mask: Tensor<f32, [32, 128]>;
    target labels: Tensor<i32, [4096]>;
    target weights: Tensor<f32, [4096]>;
    loss = cross_entropy(model.forward(ids, positions, key_mask), labels, weights);
    optimizer = adamw(lr = 1e-4, weight_decay = 0.01, beta1 = 0.9, beta2 = 0.999, eps = 1e-6, warmup_steps = 100);
    steps = 1000;
    seed = 42;
    device = hip(0);
}
