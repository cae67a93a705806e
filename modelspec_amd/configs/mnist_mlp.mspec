// The MNIST-shaped MLP without biases: 784 -> 64 (relu) -> 10, mean squared error against
// teacher data, SGD at 0.1, batches of 100.
model MnistMlp {
    param w1: Tensor<f32, [784, 64]> = xavier_uniform();
    param w2: Tensor<f32, [64, 10]> = xavier_uniform();

    fn forward(x: Tensor<f32, [100, 784]>) -> Tensor<f32, [100, 10]> {
        let hidden = relu(matmul(x, w1));
        return matmul(hidden, w2);
    }
}

train Fit {
    model = MnistMlp;
    input x: Tensor<f32, [100, 784]>;
    target y: Tensor<f32, [100, 10]>;
    loss = mse(model.forward(x), y);
    optimizer = sgd(lr = 0.1);
    steps = 1800;
    seed = 42;
    device = hip(0);
}
