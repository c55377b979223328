// The flyguy_train executable: the teaching trainer's command line, run by the library (ft_main).
extern "C" int ft_main(int argc, const char* const* argv);

int main(int argc, char** argv) { return ft_main(argc, argv); }
