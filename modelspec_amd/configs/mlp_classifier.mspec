// The MLP classifier config (BASELINE configs[1]): 784-256-10 with biases and ReLU, softmax
// cross_entropy on uniform labels with unit weights, SGD at 0.01, batches of 64, 1,000 steps.
model MlpClassifier {
    param w1: Tensor<f32, [784, 256]> = xavier_uniform();
    param b1: Tensor<f32, [256]> = zeros();
    param w2: Tensor<f32, [256, 10]> = xavier_uniform();
    param b2: Tensor<f32, [10]> = zeros();

    fn forward(x: Tensor<f32, [64, 784]>) -> Tensor<f32, [64, 10]> {
        let h = relu(add_rows(matmul(x, w1), b1));
        return add_rows(matmul(h, w2), b2);
    }
}

train Classify {
    model = MlpClassifier;
    input x: Tensor<f32, [64, 784]>;
    target labels: Tensor<i32, [64]>;
    target weights: Tensor<f32, [64]>;
    loss = cross_entropy(model.forward(x), labels, weights);
    optimizer = sgd(lr = 0.01);
    steps = 1000;
    seed = 7;
    device = hip(0);
}
